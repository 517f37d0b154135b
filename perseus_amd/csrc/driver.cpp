// The key-switching driver: the launch sequences of crates/pc-gpu restated in C++ over the kernel table.
//  - context: prime constants, twiddles and gadget scalars of one chain (crates/pc-gpu/src/context.rs:169-261);
//  - per limb top a plan (crates/pc-gpu/src/ks.rs:521-676 LevelPlan / level_specs_with): the ModUp INTT rows and their
//    N^-1 pre_t scales, the ModUp conversion jobs and NTT rows, the dot's row list, the ModDown conversion jobs, INTT
//    rows and scales, NTT rows; every table ordered [ciphertext][...] so a launch over the first m ciphertexts is a
//    prefix;
//  - key groups (crates/pc-gpu/src/ks.rs:330-400 KeyGroup; keys.rs:24-160): seeds, stored b, inverse automorphism
//    exponents;
//  - rotate (rotate.rs:179-204) and rotate_hoisted (rotate.rs:456-507).
// All device memory is allocated at setup; the per-call paths only enqueue launches on the caller's stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <new>
#include <vector>

#include "pc_hip.h"
#include "fused.h"

typedef unsigned __int128 u128;

namespace {

uint64_t mulmod(uint64_t a, uint64_t b, uint64_t m) { return (uint64_t)((u128)a * b % m); }
uint64_t powmod(uint64_t b, uint64_t e, uint64_t m) {
    uint64_t r = 1 % m;
    b %= m;
    while (e) {
        if (e & 1) r = mulmod(r, b, m);
        b = mulmod(b, b, m);
        e >>= 1;
    }
    return r;
}
uint64_t invmod(uint64_t a, uint64_t p) { return powmod(a % p, p - 2, p); }
uint32_t shoup_c(uint32_t w, uint32_t p) { return (uint32_t)(((uint64_t)w << 32) / p); }
uint32_t brev(uint32_t x, int bits) {
    uint32_t r = 0;
    for (int i = 0; i < bits; ++i) r |= ((x >> i) & 1u) << (bits - 1 - i);
    return r;
}
bool is_prime(uint64_t n) {
    if (n < 2) return false;
    static const uint64_t sp[] = {2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37};
    for (uint64_t s : sp)
        if (n % s == 0) return n == s;
    uint64_t d = n - 1;
    int s = 0;
    while (!(d & 1)) d >>= 1, ++s;
    for (uint64_t a : sp) {
        uint64_t x = powmod(a, d, n);
        if (x == 1 || x == n - 1) continue;
        bool comp = true;
        for (int i = 1; i < s && comp; ++i) {
            x = mulmod(x, x, n);
            if (x == n - 1) comp = false;
        }
        if (comp) return false;
    }
    return true;
}
// the minimal primitive m-th root of unity (crates/pc-core/src/params/nbtheory.rs:104-140)
uint64_t min_root(uint64_t m, uint64_t p) {
    uint64_t e = (p - 1) / m, w = 0;
    for (uint64_t g = 2; g < p; ++g) {
        uint64_t c = powmod(g, e, p);
        if (powmod(c, m / 2, p) == p - 1) {
            w = c;
            break;
        }
    }
    uint64_t w2 = mulmod(w, w, p), x = w, mn = w;
    for (uint64_t k = 1; k + 2 < m; k += 2) {
        x = mulmod(x, w2, p);
        if (x < mn && x != 1) mn = x;
    }
    return mn;
}
// crates/pc-core/src/modmul.rs:376-412 (word_bits 32)
PrimeConst prime_const(uint64_t p) {
    PrimeConst c;
    memset(&c, 0, sizeof c);
    c.p = p;
    c.mu_lo = (uint64_t)(((u128)1 << 64) / p);
    c.bits = 64 - __builtin_clzll(p);
    c.neal_mu = (uint64_t)(((u128)1 << (2 * c.bits + 1)) / p);
    c.word_bits = 32;
    uint64_t inv = p;
    for (int i = 0; i < 6; ++i) inv *= 2 - p * inv;
    c.mont_pinv = (-inv) & 0xFFFFFFFFull;
    c.mont_r2 = (uint64_t)(((u128)1 << 64) % p);
    uint64_t r = (1ull << 32) % p;
    c.split = r | ((r << 32) / p) << 32;
    return c;
}
// crates/pc-gpu/src/bconv.rs:34-37: pre_i = (B / b_i)^-1 mod b_i
std::vector<uint32_t> pre_factors(const std::vector<uint64_t>& bp) {
    std::vector<uint32_t> out(bp.size());
    for (size_t i = 0; i < bp.size(); ++i) {
        uint64_t h = 1;
        for (size_t k = 0; k < bp.size(); ++k)
            if (k != i) h = mulmod(h, bp[k] % bp[i], bp[i]);
        out[i] = (uint32_t)invmod(h, bp[i]);
    }
    return out;
}

struct Dev {
    std::vector<void*> owned;
    int err = 0;
    void* alloc(size_t bytes) {
        void* p = nullptr;
        if (bytes == 0) bytes = 16;
        hipError_t e = hipMalloc(&p, bytes);
        if (e != hipSuccess) {
            err = (int)e;
            return nullptr;
        }
        owned.push_back(p);
        return p;
    }
    template <class T>
    T* upload(const std::vector<T>& v) {
        T* p = (T*)alloc(v.size() * sizeof(T));
        if (p && !v.empty()) {
            hipError_t e = hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice);
            if (e != hipSuccess) err = (int)e;
        }
        return p;
    }
    ~Dev() {
        for (void* p : owned) (void)hipFree(p);
    }
};

// A fast base-conversion plan: device job records and pool (crates/pc-gpu/src/bconv.rs:59-143 build_tables)
struct JobSpec {
    uint32_t src_off, dst_off;
    std::vector<uint32_t> src, tgt;  // rows == prime ids
    bool exact = false;              // the exact conversion (the fast one corrected by u = round(sum y_i / b_i))
};
struct Bconv {
    BconvJob* jobs = nullptr;
    uint32_t* pool = nullptr;
    int njobs = 0, max_tgt = 0;
    void build(Dev& dev, const std::vector<uint64_t>& primes, const std::vector<JobSpec>& specs) {
        std::vector<uint32_t> pool_h;
        std::vector<BconvJob> jobs_h;
        for (const JobSpec& j : specs) {
            const uint32_t ns = (uint32_t)j.src.size(), nt = (uint32_t)j.tgt.size();
            BconvJob r;
            memset(&r, 0, sizeof r);
            r.src_off = j.src_off;
            r.dst_off = j.dst_off;
            r.nsrc = ns;
            r.ntgt = nt;
            r.pool_off = (uint32_t)pool_h.size();
            r.exact = j.exact ? 1 : 0;
            r.prescaled = 1;
            r.split = 0;
            std::vector<uint64_t> bp;
            for (uint32_t s : j.src) bp.push_back(primes[s]);
            for (uint32_t s : j.src) pool_h.push_back(s);
            for (uint32_t s : j.src) pool_h.push_back(s);
            for (uint32_t v : pre_factors(bp)) pool_h.push_back(v);
            for (uint32_t t : j.tgt) pool_h.push_back(t);
            for (uint32_t t : j.tgt) pool_h.push_back(t);
            for (uint32_t i = 0; i < ns; ++i)
                for (uint32_t t : j.tgt) {
                    uint64_t tp = primes[t], v = 1;
                    for (uint32_t k = 0; k < ns; ++k)
                        if (k != i) v = mulmod(v, bp[k] % tp, tp);
                    pool_h.push_back((uint32_t)v);
                }
            if (pool_h.size() & 1) pool_h.push_back(0);
            if (j.exact) {
                // rb_i = 1 / b_i as doubles (8-byte aligned: the pool's words are even here), B mod t per target, then
                // floor(2^59 / b_i) as u64 (bconv.rs:105-132)
                for (uint64_t b : bp) {
                    const double rb = 1.0 / (double)b;
                    uint64_t bits;
                    memcpy(&bits, &rb, 8);
                    pool_h.push_back((uint32_t)bits);
                    pool_h.push_back((uint32_t)(bits >> 32));
                }
                for (uint32_t t : j.tgt) {
                    uint64_t tp = primes[t], m = 1;
                    for (uint64_t b : bp) m = mulmod(m, b % tp, tp);
                    pool_h.push_back((uint32_t)m);
                }
                if (pool_h.size() & 1) pool_h.push_back(0);
                for (uint64_t b : bp) {
                    const uint64_t cq = (1ull << 59) / b;
                    pool_h.push_back((uint32_t)cq);
                    pool_h.push_back((uint32_t)(cq >> 32));
                }
            }
            jobs_h.push_back(r);
            max_tgt = std::max(max_tgt, (int)nt);
        }
        njobs = (int)jobs_h.size();
        jobs = dev.upload(jobs_h);
        pool = dev.upload(pool_h);
    }
};

struct Rows {
    uint32_t* roff = nullptr;
    int32_t* rprime = nullptr;
    uint32_t* soff = nullptr;
    uint32_t* es = nullptr;  // values then Shoup companions (W words)
    int n = 0;
};

struct Level {
    int top = 0, ndig = 0;
    Rows mu_intt;             // ModUp INTT rows (coef workspace, c1 out of place), es = N^-1 pre_t
    Bconv mu_bconv;           // per live digit: digit limbs -> the other live Q limbs and P
    Rows mu_ntt;              // the targets in the digit workspace
    uint32_t* ks_rows = nullptr;
    int nks = 0;
    // ModDown tables per chunk size m = 1..k_rot (index m - 1), prime-major so that consecutive rows share one
    // prime's twiddle table in L2: INTT of the ext P rows [j < kp][c < m][part] (es = N^-1 pre_j) and NTT of the
    // conversion's Q rows [t <= top][c < m][part]
    std::vector<Rows> md_intt;
    Bconv md_bconv;           // [c][part]: P -> Q rows 0..top (a prefix per m)
    std::vector<Rows> md_ntt;
    // the rescale from this top by one prime (index 0) or two (index 1; crates/pc-gpu/src/rescale.rs:118-160): the
    // tops' INTT rows of one ciphertext, the correction rows' NTT list (tmp rows 0..top - ndrop, both parts,
    // prime-major) and the per-prime-id constants [A | As | B | Bs | alpha | alphas | qam | qbm] (rows words each)
    struct Rescale {
        Rows intt, ntt;
        uint32_t* k = nullptr;
        uint64_t qinv_ab = 0, C_ab = 0;
    } rs[2];
    // ModDown by B = P q_top q_{top-1} at once, the rescale by the two top primes fused in (crates/pc-gpu/src/bts/
    // cts.rs:740-751, LtEnd::FusedRescale): INTT of the sources (P rows, then rows top - 1, top; both parts; es =
    // N^-1 pre_j for B), the exact conversion to rows 0..top - 2, their NTT with the epilogue (x - conv) B^-1 (es);
    // k: per row [s2 | s2 Shoup | P mod q | its Shoup] (rows words each), s2 = (q_top q_{top-1})^-1 mod q_i
    struct MdRescale {
        Rows intt, ntt;
        Bconv conv;
        uint32_t* k = nullptr;
    } mdr;
};

}  // namespace

struct pcx_rows {
    Rows r;
    Dev dev;
};

struct pcx_ctx {
    uint32_t logn = 0, n = 0;
    int nq = 0, kp = 0, dnum = 0, alpha = 0, k_rot = 1, rows = 0;
    int k_max = 1;  // ciphertexts per batched product / rescale (the per-level plans hold k_max copies)
    int lazy = 0;   // NttArgs.lazy: 1 when every prime is below 2^30 (Harvey butterflies)
    int chunk = 0;  // NttArgs.chunk of the batched transforms: rows per pass pair (0 = all)
    std::vector<uint64_t> primes, roots;
    const KernelTable* tab = nullptr;
    Dev dev;
    PrimeConst* pr = nullptr;
    uint32_t *fw = nullptr, *fws = nullptr, *iw = nullptr, *iws = nullptr, *ninv = nullptr, *ninvs = nullptr;
    uint32_t *pmod = nullptr, *pinv = nullptr;  // values then Shoup companions, by prime id
    uint32_t* mdt = nullptr;  // ModDown conversion matrix M[j][t] = [P / p_j]_{q_t}, j < kp, t < nq
    int md_fused = 1;         // ModDown conversion inside the NTT column pass (kp <= MDC_MAX_KP)
    int md_fused_init = 1;    // md_fused as chosen at creation (PCX_MD_FUSED included), restored by table_only(0)
    int table_only = 0;       // every launch through the kernel table (pcx_ctx_table_only)
    // conversions streamed into the NTT column pass (pch::conv_cols), by call site: CC_MODUP | CC_MODDOWN | CC_MDR
    // (ModDown the fused md_conv_cols does not take, the ModDown-rescale); pcx_ctx_conv_fusion, PCX_CC_FUSED. The
    // default leaves the ModDown-rescale on bconv then ntt_fwd: its exact form carries the doubles of u beside the sums
    // (2 waves per SIMD) and measured slower on the C5 bootstrap (ModUp + ModDown stages 5.09 ms unfused, 4.91 with
    // ModUp and ModDown streamed, 5.22 with the rescale's too; same box)
    int cc_fused = 3;
    int cc_tpw = 0;  // its targets per workgroup (0: from the launch's size; PCX_CC_TPW)
    int cc_ntg = 3, cc_ntgx = 2;  // targets per round of a thread's sums: fast, exact jobs (PCX_CC_NTG, PCX_CC_NTGX)
    int md_ntg = 5;           // its target rows per workgroup
    int32_t* digit_of = nullptr;
    std::vector<Level> levels;
    uint32_t *coef = nullptr, *digits = nullptr, *ext = nullptr, *conv = nullptr;
    uint32_t* tmp = nullptr;  // one ciphertext: the rescale's correction rows, a product's d2 (part 1)
    size_t ws_bytes = 0;
    // stage timing (pcx_timing): event pairs recorded around each stage's launches on the launch stream
    bool timing = false;
    std::vector<hipEvent_t> ev;
    std::vector<int> ev_stage;  // stage of pair i (events 2i, 2i + 1)
    size_t ev_used = 0;

    size_t row_words() const { return n; }
    size_t ct_words() const { return (size_t)2 * rows * n; }
    int digit(int id) const { return id < nq ? id / alpha : -1; }
};

struct pcx_keys {
    pcx_ctx* c = nullptr;
    int nkeys = 0, bits = 0;
    // the rows every key stores (crates/pc-gpu/src/keys.rs:81-103 KskShape): digits 0..ndig, each the Q rows
    // 0..=q_top then the kp special rows (srows per digit); q_top = -1: the full layout (slot = prime id)
    int q_top = -1, ndig = 0, srows = 0;
    uint64_t row_words = 0;
    std::vector<uint64_t> galois;
    std::vector<uint32_t> autok_h;
    Dev dev;
    const void** kb = nullptr;        // device array of per-key b pointers
    const uint32_t** seed = nullptr;  // device array of per-key seed pointers
    uint32_t* autok = nullptr;        // g^-1 mod 2N per key
    uint32_t* kinv = nullptr;         // g mod 2N per key (the gather exponent of a CtS baby step)
    std::vector<void*> b_ptr;         // device b storage per key
    // the KSKA retry-value table (dense keys): offsets [key][digit][row][chunk] + 1, values
    uint32_t *pidx = nullptr, *pval = nullptr;
    size_t patch_words = 0;
    std::vector<const uint32_t*> seed_ptr;  // device seed per key (host copy of `seed`)
    // resident dense `a` (pcx_keys_resident_a; crates/pc-gpu/src/ks.rs:346-347, 408-411 regen_digits): digits < regen are
    // regenerated, the rest read from ka[r] [dnum][rows][N] (prime-id rows)
    const void** ka = nullptr;
    int regen = 1 << 30;
};

namespace {

// a key group serves a ciphertext at top: every top for full keys, tops up to the band for banded ones
inline bool serves(const pcx_keys* k, int top) { return k->q_top < 0 || top <= k->q_top; }

// A stage bracket: when timing is on, an event before and after the stage's launches (stream order)
struct Stage {
    pcx_ctx* c;
    int id;
    pc_stream_t s;
    size_t slot;
    Stage(pcx_ctx* c_, int id_, pc_stream_t s_) : c(c_), id(id_), s(s_), slot(SIZE_MAX) {
        if (c->timing && 2 * (c->ev_used + 1) <= c->ev.size()) {
            slot = c->ev_used++;
            c->ev_stage[slot] = id;
            (void)hipEventRecord(c->ev[2 * slot], (hipStream_t)s);
        }
    }
    ~Stage() {
        if (slot != SIZE_MAX) (void)hipEventRecord(c->ev[2 * slot + 1], (hipStream_t)s);
    }
};

int fill_rows(Dev& dev, Rows& r, const std::vector<uint32_t>& roff, const std::vector<int32_t>& rp,
              const std::vector<uint32_t>* soff, const std::vector<uint32_t>* es) {
    r.n = (int)roff.size();
    r.roff = dev.upload(roff);
    r.rprime = dev.upload(rp);
    if (soff) r.soff = dev.upload(*soff);
    if (es) r.es = dev.upload(*es);
    return dev.err;
}

// scale tables: v[i] then shoup(v[i]) for rows of prime ids ids[i]
std::vector<uint32_t> scale_table(const std::vector<uint64_t>& primes, const std::vector<int32_t>& ids,
                                  const std::vector<uint32_t>& v) {
    std::vector<uint32_t> out(v);
    for (size_t i = 0; i < v.size(); ++i) out.push_back(shoup_c(v[i], (uint32_t)primes[ids[i]]));
    return out;
}

// the live limbs of digit d at top (crates/pc-gpu/src/ks.rs:576-578)
std::vector<uint32_t> digit_limbs(const pcx_ctx* c, int d, int top) {
    std::vector<uint32_t> v;
    for (int t = d * c->alpha; t < std::min((d + 1) * c->alpha, c->nq); ++t)
        if (t <= top) v.push_back((uint32_t)t);
    return v;
}

// The batched plans: ciphertext k's rows follow ciphertext 0's, shifted by k stride rows, so that the plan of K <= k_max
// ciphertexts is the first K / k_max of the rows (and of the conversion jobs)
template <class T>
void rep_rows(std::vector<T>& v, int kmax, int64_t stride) {
    const size_t n1 = v.size();
    for (int k = 1; k < kmax; ++k)
        for (size_t i = 0; i < n1; ++i) v.push_back((T)((int64_t)v[i] + k * stride));
}
void rep_jobs(std::vector<JobSpec>& v, int kmax, uint32_t src_stride, uint32_t dst_stride) {
    const size_t n1 = v.size();
    for (int k = 1; k < kmax; ++k)
        for (size_t i = 0; i < n1; ++i) {
            JobSpec j = v[i];
            j.src_off += (uint32_t)k * src_stride;
            j.dst_off += (uint32_t)k * dst_stride;
            v.push_back(j);
        }
}
// rows / jobs of the first K ciphertexts of a batched plan
int k_rows(const pcx_ctx* c, const Rows& r, int K) { return r.n / c->k_max * K; }
int k_jobs(const pcx_ctx* c, const Bconv& b, int K) { return b.njobs / c->k_max * K; }

int build_level(pcx_ctx* c, int top, Level& L) {
    const uint32_t n = c->n;
    const int KM = c->k_max, RR = c->rows;
    L.top = top;
    std::vector<std::vector<uint32_t>> digs;
    for (int d = 0; d < c->dnum; ++d) {
        std::vector<uint32_t> dl = digit_limbs(c, d, top);
        if (!dl.empty()) digs.push_back(dl);
    }
    L.ndig = (int)digs.size();
    // ModUp INTT: rows 0..top of the coefficient workspace, read out of place from c1, scaled by N^-1 pre_t
    std::vector<uint32_t> pre_of(top + 1);
    for (auto& dl : digs) {
        std::vector<uint64_t> bp;
        for (uint32_t t : dl) bp.push_back(c->primes[t]);
        std::vector<uint32_t> pre = pre_factors(bp);
        for (size_t k = 0; k < dl.size(); ++k) pre_of[dl[k]] = pre[k];
    }
    {
        std::vector<uint32_t> roff, soff, es;
        std::vector<int32_t> rp;
        for (int t = 0; t <= top; ++t) {
            roff.push_back(t);
            soff.push_back(t);
            rp.push_back(t);
            uint64_t p = c->primes[t];
            es.push_back((uint32_t)mulmod(invmod(n % p, p), pre_of[t], p));
        }
        // ciphertext k: coefficient rows k R + t, c1 rows k 2R + t from ciphertext 0's c1
        rep_rows(roff, KM, RR);
        rep_rows(soff, KM, 2 * RR);
        rep_rows(rp, KM, 0);
        rep_rows(es, KM, 0);
        std::vector<uint32_t> est = scale_table(c->primes, rp, es);
        if (int e = fill_rows(c->dev, L.mu_intt, roff, rp, &soff, &est)) return e;
    }
    // ModUp conversions: digit d's limbs -> (0..top minus the digit) then P, into digit d's rows of the workspace
    {
        std::vector<JobSpec> specs;
        std::vector<uint32_t> roff;
        std::vector<int32_t> rp;
        for (int d = 0; d < L.ndig; ++d) {
            JobSpec j;
            j.src_off = 0;
            j.dst_off = (uint32_t)(d * c->rows);
            j.src = digs[d];
            for (int t = 0; t <= top; ++t)
                if (std::find(digs[d].begin(), digs[d].end(), (uint32_t)t) == digs[d].end()) j.tgt.push_back(t);
            for (int k = 0; k < c->kp; ++k) j.tgt.push_back(c->nq + k);
            specs.push_back(j);
        }
        // the targets' NTT rows, prime-major (rows of one prime share its twiddle table)
        for (int t = 0; t < c->rows; ++t)
            for (int d = 0; d < L.ndig; ++d)
                if (std::find(specs[d].tgt.begin(), specs[d].tgt.end(), (uint32_t)t) != specs[d].tgt.end()) {
                    roff.push_back(specs[d].dst_off + t);
                    rp.push_back(t);
                }
        // ciphertext k: coefficient rows from k R, digit rows from k dnum R
        rep_jobs(specs, KM, (uint32_t)RR, (uint32_t)(c->dnum * RR));
        rep_rows(roff, KM, c->dnum * RR);
        rep_rows(rp, KM, 0);
        L.mu_bconv.build(c->dev, c->primes, specs);
        if (int e = fill_rows(c->dev, L.mu_ntt, roff, rp, nullptr, nullptr)) return e;
    }
    // dot rows: Q 0..top then P
    {
        std::vector<uint32_t> ks;
        for (int t = 0; t <= top; ++t) ks.push_back(t);
        for (int k = 0; k < c->kp; ++k) ks.push_back(c->nq + k);
        L.nks = (int)ks.size();
        L.ks_rows = c->dev.upload(ks);
    }
    // ModDown over up to k_rot extended ciphertexts
    {
        std::vector<uint64_t> sp;
        for (int k = 0; k < c->kp; ++k) sp.push_back(c->primes[c->nq + k]);
        std::vector<uint32_t> pre = pre_factors(sp);
        std::vector<JobSpec> specs;
        for (int ct = 0; ct < c->k_rot; ++ct)
            for (int part = 0; part < 2; ++part) {
                const uint32_t base = (uint32_t)((2 * ct + part) * c->rows);
                JobSpec j;
                j.src_off = j.dst_off = base;
                for (int k = 0; k < c->kp; ++k) j.src.push_back(c->nq + k);
                for (int t = 0; t <= top; ++t) j.tgt.push_back(t);
                specs.push_back(j);
            }
        L.md_bconv.build(c->dev, c->primes, specs);
        L.md_intt.resize(c->k_rot);
        L.md_ntt.resize(c->k_rot);
        for (int m = 1; m <= c->k_rot; ++m) {
            std::vector<uint32_t> roff, es, roff2;
            std::vector<int32_t> rp, rp2;
            for (int k = 0; k < c->kp; ++k) {
                const int id = c->nq + k;
                const uint64_t p = c->primes[id];
                const uint32_t sc = (uint32_t)mulmod(invmod(n % p, p), pre[k], p);
                for (int ct = 0; ct < m; ++ct)
                    for (int part = 0; part < 2; ++part) {
                        roff.push_back((uint32_t)((2 * ct + part) * c->rows + id));
                        rp.push_back(id);
                        es.push_back(sc);
                    }
            }
            for (int t = 0; t <= top; ++t)
                for (int ct = 0; ct < m; ++ct)
                    for (int part = 0; part < 2; ++part) {
                        roff2.push_back((uint32_t)((2 * ct + part) * c->rows + t));
                        rp2.push_back(t);
                    }
            std::vector<uint32_t> est = scale_table(c->primes, rp, es);
            if (int e = fill_rows(c->dev, L.md_intt[m - 1], roff, rp, nullptr, &est)) return e;
            if (int e = fill_rows(c->dev, L.md_ntt[m - 1], roff2, rp2, nullptr, nullptr)) return e;
        }
    }
    // rescale by one or two primes: qlql[l][i] = -q_l^-1 mod q_i, qinv[l][i] = q_l^-1 mod q_i
    // (crates/pc-core/src/scale.rs:196-208); ndrop 1: A_i = qlql[a][i], alpha_i = qinv[a][i]; ndrop 2 (a = top,
    // b = top - 1): A_i = qinv[b][i] qlql[a][i], B_i = qlql[b][i], alpha_i = qinv[b][i] qinv[a][i]
    for (int g = 1; g <= 2; ++g) {
        if (top < g) continue;
        Level::Rescale& Z = L.rs[g - 1];
        const int a = top, b = top - 1, R = c->rows;
        auto qinv = [&](int l, int i) { return invmod(c->primes[l] % c->primes[i], c->primes[i]); };
        auto qlql = [&](int l, int i) {
            const uint64_t v = qinv(l, i);
            return v ? c->primes[i] - v : 0;
        };
        std::vector<uint32_t> k((size_t)8 * R, 0);
        for (int i = 0; i + g <= top; ++i) {
            const uint64_t qi = c->primes[i];
            uint64_t A, B = 0, al;
            if (g == 1) {
                A = qlql(a, i);
                al = qinv(a, i);
            } else {
                A = mulmod(qinv(b, i), qlql(a, i), qi);
                B = qlql(b, i);
                al = mulmod(qinv(b, i), qinv(a, i), qi);
            }
            k[0 * R + i] = (uint32_t)A;
            k[1 * R + i] = shoup_c((uint32_t)A, (uint32_t)qi);
            k[2 * R + i] = (uint32_t)B;
            k[3 * R + i] = shoup_c((uint32_t)B, (uint32_t)qi);
            k[4 * R + i] = (uint32_t)al;
            k[5 * R + i] = shoup_c((uint32_t)al, (uint32_t)qi);
            k[6 * R + i] = (uint32_t)(c->primes[a] % qi);
            k[7 * R + i] = (uint32_t)(c->primes[b] % qi);
        }
        if (g == 2) {
            Z.qinv_ab = qinv(a, b);
            Z.C_ab = qlql(a, b);
        }
        Z.k = c->dev.upload(k);
        std::vector<uint32_t> roff, roff2;
        std::vector<int32_t> rp, rp2;
        for (int t = top + 1 - g; t <= top; ++t)
            for (int part = 0; part < 2; ++part) {
                roff.push_back((uint32_t)(part * R + t));
                rp.push_back(t);
            }
        for (int t = 0; t + g <= top; ++t)
            for (int part = 0; part < 2; ++part) {
                roff2.push_back((uint32_t)(part * R + t));
                rp2.push_back(t);
            }
        // ciphertext k (and its correction rows in tmp) at k 2R rows
        rep_rows(roff, KM, 2 * R);
        rep_rows(rp, KM, 0);
        rep_rows(roff2, KM, 2 * R);
        rep_rows(rp2, KM, 0);
        if (int e = fill_rows(c->dev, Z.intt, roff, rp, nullptr, nullptr)) return e;
        if (int e = fill_rows(c->dev, Z.ntt, roff2, rp2, nullptr, nullptr)) return e;
    }
    if (top >= 2) {
        const int R = c->rows;
        std::vector<uint32_t> src;
        for (int k = 0; k < c->kp; ++k) src.push_back((uint32_t)(c->nq + k));
        src.push_back((uint32_t)(top - 1));
        src.push_back((uint32_t)top);
        std::vector<uint64_t> bp;
        for (uint32_t id : src) bp.push_back(c->primes[id]);
        const std::vector<uint32_t> pre = pre_factors(bp);
        std::vector<uint32_t> roff, es, roff2, bi;
        std::vector<int32_t> rp, rp2;
        for (size_t j = 0; j < src.size(); ++j) {
            const uint64_t p = bp[j];
            const uint32_t sc = (uint32_t)mulmod(invmod(n % p, p), pre[j], p);
            for (int part = 0; part < 2; ++part) {
                roff.push_back((uint32_t)(part * R) + src[j]);
                rp.push_back((int32_t)src[j]);
                es.push_back(sc);
            }
        }
        std::vector<JobSpec> specs;
        for (int part = 0; part < 2; ++part) {
            JobSpec j;
            j.src_off = j.dst_off = (uint32_t)(part * R);
            j.src = src;
            for (int t = 0; t + 2 <= top; ++t) j.tgt.push_back((uint32_t)t);
            j.exact = true;
            specs.push_back(j);
        }
        // the epilogue's B^-1 by prime id (rows of other ids unused)
        std::vector<uint32_t> binv(R, 0), k((size_t)4 * R, 0);
        for (int t = 0; t + 2 <= top; ++t) {
            const uint64_t q = c->primes[t];
            uint64_t b = 1;
            for (uint64_t x : bp) b = mulmod(b, x % q, q);
            binv[t] = (uint32_t)invmod(b, q);
            const uint32_t s2 = (uint32_t)invmod(mulmod(c->primes[top] % q, c->primes[top - 1] % q, q), q);
            k[t] = s2;
            k[R + t] = shoup_c(s2, (uint32_t)q);
            for (int part = 0; part < 2; ++part) {
                roff2.push_back((uint32_t)(part * R + t));
                rp2.push_back(t);
            }
        }
        for (int t = top - 1; t <= top; ++t) {
            const uint64_t q = c->primes[t];
            uint64_t pm = 1;
            for (int j = 0; j < c->kp; ++j) pm = mulmod(pm, c->primes[c->nq + j] % q, q);
            k[2 * R + t] = (uint32_t)pm;
            k[3 * R + t] = shoup_c((uint32_t)pm, (uint32_t)q);
        }
        // ciphertext k's extended rows, conversion rows and output rows at k 2R
        rep_rows(roff, KM, 2 * R);
        rep_rows(rp, KM, 0);
        rep_rows(es, KM, 0);
        rep_rows(roff2, KM, 2 * R);
        rep_rows(rp2, KM, 0);
        rep_jobs(specs, KM, (uint32_t)(2 * R), (uint32_t)(2 * R));
        std::vector<uint32_t> est = scale_table(c->primes, rp, es);
        std::vector<int32_t> ids(R);
        for (int i = 0; i < R; ++i) ids[i] = i;
        std::vector<uint32_t> bt = scale_table(c->primes, ids, binv);
        if (int e = fill_rows(c->dev, L.mdr.intt, roff, rp, nullptr, &est)) return e;
        if (int e = fill_rows(c->dev, L.mdr.ntt, roff2, rp2, nullptr, &bt)) return e;
        L.mdr.conv.build(c->dev, c->primes, specs);
        L.mdr.k = c->dev.upload(k);
    }
    return c->dev.err;
}

NttArgs ntt_args(const pcx_ctx* c, void* base, const Rows& r, int nrows) {
    NttArgs a;
    memset(&a, 0, sizeof a);
    a.base = base;
    a.roff = r.roff;
    a.rprime = r.rprime;
    a.fw = c->fw;
    a.fws = c->fws;
    a.iw = c->iw;
    a.iws = c->iws;
    a.ninv = c->ninv;
    a.ninvs = c->ninvs;
    a.pr = c->pr;
    a.nrows = nrows;
    a.chunk = c->chunk;
    a.lazy = c->lazy;
    a.snum = 1;
    a.xnum = 1;
    return a;
}

const Level* level(const pcx_ctx* c, int top) {
    if (top < 0 || top >= c->nq) return nullptr;
    return &c->levels[top];
}

enum { CC_MODUP = 1, CC_MODDOWN = 2, CC_MDR = 4 };
bool cc_on(const pcx_ctx* c, int site) { return !c->table_only && (c->cc_fused & site); }
// targets per round (returned) and per workgroup (tpw) of a streamed conversion of jobs of at most nsrc sources:
// ntg0 targets per round, fewer (down to 1) for jobs of at most 8 sources when one round per workgroup leaves the
// launch under about 2048 workgroups (a small launch then spreads its targets over more CUs: a C1 rotation 0.0592 ->
// 0.0548 ms beside the ModDown's own fewer rows per workgroup, while the bootstrap's 16-source jobs lost more to
// re-reading their sources than they gained),
// then rounds per workgroup raised while the launch keeps about 2048 workgroups (each target group re-reads its
// column block's sources from L2)
int cc_shape(const pcx_ctx* c, const BconvArgs& b, int ntg0, int nsrc, int* tpw) {
    if (c->cc_tpw > 0) {
        *tpw = c->cc_tpw;
        return ntg0;
    }
    const long per = (long)(c->n / 4096) * b.njobs;
    int ntg = ntg0;
    while (nsrc <= 8 && ntg > 1 && per * ((b.max_tgt + ntg - 1) / ntg) < 2048) --ntg;
    int k = 1;
    while (k < 4 && per * ((b.max_tgt + ntg * (k + 1) - 1) / (ntg * (k + 1))) >= 2048) ++k;
    *tpw = ntg * k;
    return ntg;
}
// the conversion b streamed into the column pass of f's rows (exactly b's targets), then f's row pass and epilogue
// (exact: b's jobs are the exact conversion)
int conv_then_rows(pcx_ctx* c, const BconvArgs& b, const NttArgs& f, pc_stream_t s, int st_conv, int st_rows,
                   int nsrc, int exact = 0) {
    {
        Stage st(c, st_conv, s);
        int tpw = 0;
        const int ntg = cc_shape(c, b, exact ? c->cc_ntgx : c->cc_ntg, nsrc, &tpw);
        if (int e = pch::conv_cols((int)c->logn, &b, c->fw, c->fws, c->lazy, exact, ntg, tpw, s)) return e;
    }
    Stage st(c, st_rows, s);
    return pch::ntt_fwd_rows_only((int)c->logn, &f, s);
}

// ModUp (crates/pc-gpu/src/ks.rs:958-1040): INTT of c1 rows 0..top (out of place, N^-1 pre_t), conversion of every
// live digit, NTT of the targets
// ModDown and the two-prime rescale at once (the level's mdr plan): out (Q rows 0..top - 2) = the exact
// (x + P onto - conv_B) / B with B = P q_top q_{top-1}, x = ext (one extended ciphertext), onto NULL or a ciphertext at
// top (may alias out)
// K <= k_max ciphertexts at once: ext, out and onto each K consecutive ciphertexts (ct_words apart)
// nsum > 1 (K = 1): x is the sum of nsum extended ciphertexts ct_words apart (the INTT's first pass and the epilogue
// read the sum; onto's P multiple goes into the first)
int moddown_rescale(pcx_ctx* c, void* ext, int top, void* out, const void* onto, pc_stream_t s, int K = 1,
                    int nsum = 1) {
    const Level* L = level(c, top);
    if (!L || top < 2 || !L->mdr.k || K < 1 || K > c->k_max || nsum < 1 || (nsum > 1 && K != 1)) return -1;
    const Level::MdRescale& M = L->mdr;
    if (onto) {
        Stage st(c, 9, s);
        if (int e = pch::mdr_prep((int)c->logn, ext, onto, out, M.k, c->pr, c->rows, top, K, s)) return e;
    }
    NttArgs a = ntt_args(c, ext, M.intt, k_rows(c, M.intt, K));
    a.es = M.intt.es;
    a.ess = M.intt.es + M.intt.n;
    if (nsum > 1) {
        a.src = ext;
        a.soff = M.intt.roff;
        a.snum = nsum;
        a.sstride = c->ct_words();
    }
    {
        Stage st(c, 4, s);
        if (int e = c->tab->ntt_inv(&a, s)) return e;
    }
    BconvArgs b;
    memset(&b, 0, sizeof b);
    b.src = ext;
    b.dst = c->conv;
    b.jobs = M.conv.jobs;
    b.pool = M.conv.pool;
    b.pr = c->pr;
    b.njobs = k_jobs(c, M.conv, K);
    b.max_tgt = M.conv.max_tgt;
    NttArgs f = ntt_args(c, c->conv, M.ntt, k_rows(c, M.ntt, K));
    f.epi = onto ? 2 : 1;
    f.ed = nullptr;  // the epilogue adds onto out's rows, which hold onto s2
    f.eout = out;
    f.ex = ext;
    f.xnum = nsum;
    f.xstride = c->ct_words();
    f.es = M.ntt.es;
    f.ess = M.ntt.es + c->rows;
    if (cc_on(c, CC_MDR)) return conv_then_rows(c, b, f, s, 5, 6, c->kp + 2, 1);
    {
        Stage st(c, 5, s);
        if (int e = c->tab->bconv(&b, s)) return e;
    }
    Stage st(c, 6, s);
    return c->tab->ntt_fwd(&f, s);
}
// K <= k_max consecutive ciphertexts (ct_words apart): digits of ciphertext k at digits + k dnum rows N
int modup(pcx_ctx* c, const void* ct, int top, pc_stream_t s, int K = 1) {
    const Level* L = level(c, top);
    if (!L || K < 1 || K > c->k_max) return -1;
    NttArgs a = ntt_args(c, c->coef, L->mu_intt, k_rows(c, L->mu_intt, K));
    a.src = (const uint32_t*)ct + (size_t)c->rows * c->n;  // c1
    a.soff = L->mu_intt.soff;
    a.snum = 1;
    a.es = L->mu_intt.es;
    a.ess = L->mu_intt.es + L->mu_intt.n;
    {
        Stage st(c, 0, s);
        if (int e = c->tab->ntt_inv(&a, s)) return e;
    }
    BconvArgs b;
    memset(&b, 0, sizeof b);
    b.src = c->coef;
    b.dst = c->digits;
    b.jobs = L->mu_bconv.jobs;
    b.pool = L->mu_bconv.pool;
    b.pr = c->pr;
    b.njobs = k_jobs(c, L->mu_bconv, K);
    b.max_tgt = L->mu_bconv.max_tgt;
    NttArgs f = ntt_args(c, c->digits, L->mu_ntt, k_rows(c, L->mu_ntt, K));
    if (cc_on(c, CC_MODUP)) return conv_then_rows(c, b, f, s, 1, 2, c->alpha);
    {
        Stage st(c, 1, s);
        if (int e = c->tab->bconv(&b, s)) return e;
    }
    Stage st(c, 2, s);
    return c->tab->ntt_fwd(&f, s);
}

// the dot of keys [r0, r0 + m) of k into m extended ciphertexts at ext (crates/pc-gpu/src/ks.rs:1225-1308 dot_key);
// sum: 1 sums the m rotations into ext's first ciphertext (KS_SUM), 2 adds that sum onto it (KS_SUM | KS_ACC)
// K consecutive ciphertexts (ct_words apart, their digits dnum rows N apart) against the same keys: extended
// ciphertext (k, r) at ext + (k m + r) ct_words
int dot(pcx_ctx* c, pcx_keys* k, int r0, int m, const void* ct, int top, void* ext, pc_stream_t s, int sum = 0,
        int c0_mode = 1, int K = 1, const uint32_t* digits = nullptr, const void* c0 = nullptr) {
    const Level* L = level(c, top);
    if (!L || r0 < 0 || m < 1 || r0 + m > k->nkeys || K < 1 || K > c->k_max || K > 4) return -1;
    if (k->q_top >= 0 && top > k->q_top) return -1;  // above the keys' band
    KsKeyArgs g;
    memset(&g, 0, sizeof g);
    KsArgs& a = g.ks;
    a.c1 = (const uint32_t*)ct + (size_t)c->rows * c->n;
    a.modup = digits ? digits : c->digits;
    a.c0 = c0 ? c0 : ct;
    a.out0 = ext;
    a.out1 = (uint32_t*)ext + (size_t)c->rows * c->n;
    a.kb = nullptr;
    a.ka = nullptr;
    a.autok = k->autok + r0;
    a.rows = L->ks_rows;
    a.digit_of = c->digit_of;
    a.pmod = c->pmod;
    a.pmods = c->pmod + (c->nq + c->kp);
    a.pr = c->pr;
    a.ct_stride = c->ct_words();
    a.mu_ct_stride = (uint64_t)c->dnum * c->rows * c->n;
    a.mu_digit_stride = (uint64_t)c->rows * c->n;
    a.out_ct_stride = (uint64_t)(sum ? 1 : m) * c->ct_words();  // a sum: one extended ciphertext per ciphertext
    a.out_rot_stride = c->ct_words();
    a.key_digit_stride = 0;
    a.K = K;
    a.R = m;
    a.ndig = L->ndig;
    a.c0_mode = c0_mode | (sum ? PC_KS_SUM : 0) | (sum == 2 ? PC_KS_ACC : 0);
    a.nq = c->nq;
    a.nrows = L->nks;
    KeyTab& t = g.key;
    t.kb = k->kb + r0;
    t.seed = k->seed + r0;
    t.row_words = k->row_words;
    t.bits = k->bits;
    t.q_top = k->q_top;
    t.srows = k->srows;
    t.nregen = k->ndig;
    if (k->ka && k->regen < L->ndig) {
        // the keys' resident `a` for digits >= regen
        t.nregen = k->regen;
        a.ka = k->ka + r0;
        a.key_digit_stride = (uint64_t)c->rows * c->n;
    }
    Stage st(c, 3, s);
    if (k->pval && !sum && !c->table_only) {
        // the retry values from the key group's table (no redraw in the dot)
        // the table is indexed by the group's key: the launch's key r is the group's r0 + r
        const size_t per_key = (size_t)c->dnum * c->rows * (c->n / 1024);
        const pch::PatchTab P = {k->pidx + (size_t)r0 * per_key, k->pval, c->dnum, c->rows};
        const int rc = pch::ks_dot_patched((int)c->logn, &g, &P, s);
        if (rc != -2) return rc;
    }
    return c->tab->ks_dot_key(&g, s);
}

// ModDown of m extended ciphertexts at ext into m ciphertexts at out (crates/pc-gpu/src/ks.rs:1620-1649): INTT of the
// P rows (N^-1 pre_j), conversion P -> Q rows 0..top into conv, NTT of conv with the epilogue (ext - conv) P^-1;
// onto non-null: onto + (ext - conv) P^-1 (onto == out: added in place; crates/pc-gpu/src/ks.rs:1675-1710 MdOut)
// the dots of m consecutive inputs (ct_words apart, their digits at digits, dnum rows N apart), input j under key
// r0 + j alone, into m extended ciphertexts at ext (ct_words apart), each c0 folded in as P sigma_j(c0_j): one launch
// of the fast dot's diagonal form (the key group's retry table); -2 where that form does not apply
int dot_diag(pcx_ctx* c, pcx_keys* k, int r0, int m, const void* ct, int top, void* ext, const uint32_t* digits,
             pc_stream_t s) {
    const Level* L = level(c, top);
    if (!L || r0 < 0 || m < 1 || r0 + m > k->nkeys || m > c->k_max) return -1;
    if (!k->pval || c->table_only || k->q_top >= 0) return -2;
    KsKeyArgs g;
    memset(&g, 0, sizeof g);
    KsArgs& a = g.ks;
    a.c1 = (const uint32_t*)ct + (size_t)c->rows * c->n;
    a.modup = digits;
    a.c0 = ct;
    a.out0 = ext;
    a.out1 = (uint32_t*)ext + (size_t)c->rows * c->n;
    a.autok = k->autok + r0;
    a.rows = L->ks_rows;
    a.digit_of = c->digit_of;
    a.pmod = c->pmod;
    a.pmods = c->pmod + (c->nq + c->kp);
    a.pr = c->pr;
    a.ct_stride = c->ct_words();
    a.mu_ct_stride = (uint64_t)c->dnum * c->rows * c->n;
    a.mu_digit_stride = (uint64_t)c->rows * c->n;
    a.out_ct_stride = c->ct_words();
    a.out_rot_stride = 0;
    a.K = m;
    a.R = m;
    a.ndig = L->ndig;
    a.c0_mode = 1;
    a.nq = c->nq;
    a.nrows = L->nks;
    KeyTab& t = g.key;
    t.kb = k->kb + r0;
    t.seed = k->seed + r0;
    t.row_words = k->row_words;
    t.bits = k->bits;
    t.q_top = -1;
    t.srows = c->rows;
    t.nregen = c->dnum;
    Stage st(c, 3, s);
    const size_t per_key = (size_t)c->dnum * c->rows * (c->n / 1024);
    const pch::PatchTab P = {k->pidx + (size_t)r0 * per_key, k->pval, c->dnum, c->rows, 1};
    return pch::ks_dot_patched((int)c->logn, &g, &P, s);
}

// nsum > 1 (m = 1): ext holds nsum extended ciphertexts ct_words apart, the ModDown of their sum
int moddown(pcx_ctx* c, void* ext, uint32_t* conv, int m, int top, void* out, pc_stream_t s,
            const void* onto = nullptr, int nsum = 1) {
    const Level* L = level(c, top);
    if (!L || m < 1 || m > c->k_rot || nsum < 1 || (nsum > 1 && m != 1)) return -1;
    const Rows& ri = L->md_intt[m - 1];
    NttArgs a = ntt_args(c, ext, ri, ri.n);
    a.es = ri.es;
    a.ess = ri.es + ri.n;
    if (nsum > 1) {
        a.src = ext;
        a.soff = ri.roff;
        a.snum = nsum;
        a.sstride = c->ct_words();
    }
    {
        Stage st(c, 4, s);
        if (int e = c->tab->ntt_inv(&a, s)) return e;
    }
    const Rows& rn = L->md_ntt[m - 1];
    NttArgs f = ntt_args(c, conv, rn, rn.n);
    f.epi = onto ? 2 : 1;
    f.ed = onto == out ? nullptr : onto;
    f.eout = out;
    f.ex = ext;
    f.xnum = nsum;
    f.xstride = c->ct_words();
    f.es = c->pinv;
    f.ess = c->pinv + (c->nq + c->kp);
    if (c->md_fused) {
        // the conversion inside the NTT's column pass, then the row pass with the epilogue
        pch::MdcArgs d;
        d.ext = (const uint32_t*)ext;
        d.conv = conv;
        d.mt = c->mdt;
        d.pr = c->pr;
        d.fw = c->fw;
        d.fws = c->fws;
        d.nq = c->nq;
        d.kp = c->kp;
        d.rows = c->rows;
        d.top = top;
        d.ntg = c->md_ntg;
        d.m = m;
        d.lazy = c->lazy;
        {
            Stage st(c, 5, s);
            if (int e = pch::md_conv_cols((int)c->logn, &d, s)) return e;
        }
        Stage st(c, 6, s);
        return pch::ntt_fwd_rows_only((int)c->logn, &f, s);
    }
    BconvArgs b;
    memset(&b, 0, sizeof b);
    b.src = ext;
    b.dst = conv;
    b.jobs = L->md_bconv.jobs;
    b.pool = L->md_bconv.pool;
    b.pr = c->pr;
    b.njobs = 2 * m;
    b.max_tgt = top + 1;
    if (cc_on(c, CC_MODDOWN)) return conv_then_rows(c, b, f, s, 5, 6, c->kp);
    {
        Stage st(c, 5, s);
        if (int e = c->tab->bconv(&b, s)) return e;
    }
    Stage st(c, 6, s);
    return c->tab->ntt_fwd(&f, s);
}

// out = a + b on Q rows 0..top of both parts (the table's ew_add)
int add_q(pcx_ctx* c, const void* a, const void* b, int top, void* out, pc_stream_t s) {
    const uint64_t part = (uint64_t)c->rows * c->n;
    EwArgs e;
    memset(&e, 0, sizeof e);
    e.out = PolyRef{out, 0, part};
    e.a = PolyRef{const_cast<void*>(a), 0, part};
    e.b = PolyRef{const_cast<void*>(b), 0, part};
    e.rs = RowSet{top + 1, 0, 0, 0};
    e.pr = c->pr;
    e.K = 1;
    e.nparts = 2;
    return c->tab->ew_add(&e, s);
}

// the identity rotation: Q rows 0..top of both parts, one launch of the table's ew_copy
int copy_q(pcx_ctx* c, const void* ct, int top, void* out, pc_stream_t s, int K = 1) {
    const uint64_t part = (uint64_t)c->rows * c->n;
    EwArgs a;
    memset(&a, 0, sizeof a);
    a.out = PolyRef{out, 2 * part, part};
    a.a = PolyRef{const_cast<void*>(ct), 2 * part, part};
    a.rs = RowSet{top + 1, 0, 0, 0};
    a.pr = c->pr;
    a.K = K;
    a.nparts = 2;
    return c->tab->ew_copy(&a, s);
}

void pack_row(const uint32_t* v, uint32_t n, int bits, uint32_t* out, uint64_t row_words) {
    memset(out, 0, row_words * 4);
    for (uint32_t i = 0; i < n; ++i) {
        const uint64_t bit = (uint64_t)i * bits;
        const uint64_t w = bit >> 5, off = bit & 31;
        const uint64_t x = (uint64_t)v[i] << off;
        out[w] |= (uint32_t)x;
        if (off + bits > 32) out[w + 1] |= (uint32_t)(x >> 32);
    }
}

uint64_t packed_row_words(uint32_t n, int bits) {
    // crates/pc-gpu/src/keys.rs:54-58: N bits / 32 words, one zero guard word, padded to 16 bytes
    return ((uint64_t)n * bits / 32 + 1 + 3) / 4 * 4;
}

pcx_keys* keys_shell(pcx_ctx* c, int nkeys, const uint64_t* galois, int bits, int* err) {
    if (nkeys < 1 || bits < 0 || bits > 32 || (bits > 0 && bits < 31 && false)) {
        *err = -1;
        return nullptr;
    }
    for (int i = 0; i < c->nq + c->kp; ++i)
        if (bits > 0 && (c->primes[i] >> bits) != 0) {
            *err = -1;  // a prime wider than the packed width
            return nullptr;
        }
    pcx_keys* k = new (std::nothrow) pcx_keys;
    if (!k) {
        *err = -1;
        return nullptr;
    }
    k->c = c;
    k->nkeys = nkeys;
    k->bits = bits;
    k->ndig = c->dnum;
    k->srows = c->rows;
    k->row_words = bits ? packed_row_words(c->n, bits) : c->n;
    const uint64_t m = 2ull * c->n;
    for (int r = 0; r < nkeys; ++r) {
        uint64_t g = galois[r] % m;
        if (!(g & 1)) {
            delete k;
            *err = -1;
            return nullptr;
        }
        k->galois.push_back(g);
        k->autok_h.push_back((uint32_t)powmod(g, (m >> 2) - 1, m));  // g^-1 (crates/pc-core/src/galois.rs:50-59)
    }
    k->autok = k->dev.upload(k->autok_h);
    std::vector<uint32_t> gh(k->galois.begin(), k->galois.end());
    k->kinv = k->dev.upload(gh);
    if (!k->autok || !k->kinv) {
        *err = k->dev.err ? k->dev.err : -1;
        delete k;
        return nullptr;
    }
    return k;
}

// The retry-value table of a dense key group (a kernel counts each chunk's rejected KSKA words, the host takes the
// exclusive prefix, a second kernel writes the redrawn values); skipped when PCX_KS_PATCH=0
int build_patches(pcx_ctx* c, pcx_keys* k) {
    if (k->bits != 0) return 0;
    if (const char* e = getenv("PCX_KS_PATCH"))
        if (atoi(e) == 0) return 0;
    const size_t chunks = c->n / 1024, cells = (size_t)k->nkeys * c->dnum * c->rows * chunks;
    uint32_t* cnt = (uint32_t*)k->dev.alloc(cells * 4);
    if (!cnt) return k->dev.err;
    if (int e = pch::kska_patch_count((int)c->logn, k->seed, c->pr, k->nkeys, c->dnum, c->rows, cnt, nullptr)) return e;
    std::vector<uint32_t> h(cells);
    if (hipMemcpy(h.data(), cnt, cells * 4, hipMemcpyDeviceToHost) != hipSuccess) return -1;
    std::vector<uint32_t> off(cells + 1);
    uint64_t acc = 0;
    for (size_t i = 0; i < cells; ++i) {
        off[i] = (uint32_t)acc;
        acc += h[i];
    }
    if (acc >= 0xFFFFFFFFull) return -1;
    off[cells] = (uint32_t)acc;
    k->pidx = k->dev.upload(off);
    k->pval = (uint32_t*)k->dev.alloc(std::max<uint64_t>(acc, 1) * 4);
    if (!k->pidx || !k->pval) return k->dev.err ? k->dev.err : -1;
    if (int e = pch::kska_patch_fill((int)c->logn, k->seed, c->pr, k->nkeys, c->dnum, c->rows, k->pidx, k->pval,
                                     nullptr))
        return e;
    if (hipDeviceSynchronize() != hipSuccess) return -1;
    k->patch_words = (cells + 1) + acc;
    return 0;
}

}  // namespace

extern "C" {

pcx_ctx* pcx_ctx_new(uint32_t log_n, const uint64_t* primes, int nq, int kp, int dnum, int k_rot, int* err) {
    return pcx_ctx_new_k(log_n, primes, nq, kp, dnum, k_rot, 1, err);
}
pcx_ctx* pcx_ctx_new_k(uint32_t log_n, const uint64_t* primes, int nq, int kp, int dnum, int k_rot, int k_max,
                       int* err) {
    int dummy;
    if (!err) err = &dummy;
    *err = 0;
    const KernelTable* tab = pc_table_u32_logn(log_n);
    if (!tab || nq < 1 || kp < 1 || dnum < 1 || dnum > nq || k_rot < 1 || k_max < 1 || k_max > 8 || !primes) {
        *err = -1;
        return nullptr;
    }
    const uint32_t n = 1u << log_n;
    for (int i = 0; i < nq + kp; ++i) {
        uint64_t p = primes[i];
        if (p >= (1ull << 31) || p < 3 || (p - 1) % (2ull * n) || !is_prime(p)) {
            *err = -1;
            return nullptr;
        }
        for (int k = 0; k < i; ++k)
            if (primes[k] == p) {
                *err = -1;
                return nullptr;
            }
    }
    pcx_ctx* c = new (std::nothrow) pcx_ctx;
    if (!c) {
        *err = -1;
        return nullptr;
    }
    c->logn = log_n;
    c->n = n;
    c->nq = nq;
    c->kp = kp;
    c->dnum = dnum;
    c->alpha = (nq + dnum - 1) / dnum;
    c->k_rot = k_rot;
    c->k_max = k_max;
    c->rows = nq + kp;
    c->tab = tab;
    c->primes.assign(primes, primes + nq + kp);
    c->lazy = std::all_of(c->primes.begin(), c->primes.end(), [](uint64_t p) { return p < (1ull << 30); }) ? 1 : 0;
    // rows per NTT pass pair (0: one pass pair over all rows, measured fastest; PCX_NTT_CHUNK overrides)
    c->chunk = 0;
    if (const char* e = getenv("PCX_NTT_CHUNK")) c->chunk = atoi(e);
    c->md_fused = kp <= pch::MDC_MAX_KP ? 1 : 0;
    if (const char* e = getenv("PCX_MD_FUSED")) c->md_fused = c->md_fused && atoi(e) != 0;
    c->md_fused_init = c->md_fused;
    if (const char* e = getenv("PCX_CC_FUSED")) c->cc_fused = atoi(e) & 7;
    if (const char* e = getenv("PCX_CC_TPW")) c->cc_tpw = std::max(0, atoi(e));
    if (const char* e = getenv("PCX_CC_NTG")) c->cc_ntg = std::max(1, std::min(3, atoi(e)));
    if (const char* e = getenv("PCX_CC_NTGX")) c->cc_ntgx = std::max(1, std::min(3, atoi(e)));
    if (const char* e = getenv("PCX_MD_NTG")) c->md_ntg = std::max(1, std::min(pch::MDC_MAX_NTG, atoi(e)));
    const int R = c->rows;
    // prime constants and twiddles (crates/pc-gpu/src/context.rs:186-230)
    std::vector<PrimeConst> pc;
    std::vector<uint32_t> fw((size_t)R * n), fws((size_t)R * n), iw((size_t)R * n), iws((size_t)R * n);
    std::vector<uint32_t> ninv, ninvs;
    for (int id = 0; id < R; ++id) {
        const uint64_t p = c->primes[id];
        pc.push_back(prime_const(p));
        const uint64_t psi = min_root(2ull * n, p), ipsi = invmod(psi, p);
        c->roots.push_back(psi);
        uint64_t x = 1, y = 1;
        std::vector<uint32_t> pw(n), ipw(n);
        for (uint32_t i = 0; i < n; ++i) {
            pw[i] = (uint32_t)x;
            ipw[i] = (uint32_t)y;
            x = mulmod(x, psi, p);
            y = mulmod(y, ipsi, p);
        }
        for (uint32_t i = 0; i < n; ++i) {
            const uint32_t e = brev(i, log_n);
            const size_t o = (size_t)id * n + i;
            fw[o] = pw[e];
            fws[o] = shoup_c(pw[e], (uint32_t)p);
            iw[o] = ipw[e];
            iws[o] = shoup_c(ipw[e], (uint32_t)p);
        }
        ninv.push_back((uint32_t)invmod(n % p, p));
        ninvs.push_back(shoup_c(ninv.back(), (uint32_t)p));
    }
    c->pr = c->dev.upload(pc);
    c->fw = c->dev.upload(fw);
    c->fws = c->dev.upload(fws);
    c->iw = c->dev.upload(iw);
    c->iws = c->dev.upload(iws);
    c->ninv = c->dev.upload(ninv);
    c->ninvs = c->dev.upload(ninvs);
    // P mod q and P^-1 mod q by prime id, then their Shoup companions (crates/pc-gpu/src/context.rs:234-259)
    std::vector<uint32_t> pm(R, 0), pi(R, 0);
    for (int t = 0; t < nq; ++t) {
        uint64_t q = c->primes[t], m = 1;
        for (int k = 0; k < kp; ++k) m = mulmod(m, c->primes[nq + k] % q, q);
        pm[t] = (uint32_t)m;
        pi[t] = (uint32_t)invmod(m, q);
    }
    std::vector<uint32_t> pm2(pm), pi2(pi);
    for (int t = 0; t < R; ++t) {
        pm2.push_back(shoup_c(pm[t], (uint32_t)c->primes[t]));
        pi2.push_back(shoup_c(pi[t], (uint32_t)c->primes[t]));
    }
    c->pmod = c->dev.upload(pm2);
    c->pinv = c->dev.upload(pi2);
    {
        std::vector<uint32_t> mt((size_t)kp * nq);
        for (int jj = 0; jj < kp; ++jj)
            for (int t = 0; t < nq; ++t) {
                const uint64_t q = c->primes[t];
                uint64_t v = 1;
                for (int k = 0; k < kp; ++k)
                    if (k != jj) v = mulmod(v, c->primes[nq + k] % q, q);
                mt[(size_t)jj * nq + t] = (uint32_t)v;
            }
        c->mdt = c->dev.upload(mt);
    }
    std::vector<int32_t> dof(R);
    for (int t = 0; t < R; ++t) dof[t] = c->digit(t);
    c->digit_of = c->dev.upload(dof);
    c->levels.resize(nq);
    for (int top = 0; top < nq && !c->dev.err; ++top)
        if (int e = build_level(c, top, c->levels[top])) {
            *err = e;
            delete c;
            return nullptr;
        }
    // workspace: coefficient rows and ModUp digits of k_max ciphertexts, max(k_rot, k_max) extended ciphertexts and
    // their conversions, k_max ciphertexts of products' d2 and rescale corrections
    const size_t rw = (size_t)n * 4, next = (size_t)std::max(k_rot, k_max);
    const size_t coef_rows = k_max == 1 ? (size_t)nq : (size_t)k_max * R;
    c->coef = (uint32_t*)c->dev.alloc(coef_rows * rw);
    c->digits = (uint32_t*)c->dev.alloc((size_t)k_max * dnum * R * rw);
    c->ext = (uint32_t*)c->dev.alloc(next * 2 * R * rw);
    c->conv = (uint32_t*)c->dev.alloc(next * 2 * R * rw);
    c->tmp = (uint32_t*)c->dev.alloc((size_t)k_max * 2 * R * rw);
    c->ws_bytes = (coef_rows + (size_t)k_max * dnum * R + 2 * next * 2 * R + (size_t)k_max * 2 * R) * rw;
    if (c->dev.err) {
        *err = c->dev.err;
        delete c;
        return nullptr;
    }
    if (hipMemset(c->digits, 0, (size_t)k_max * dnum * R * rw) != hipSuccess) c->dev.err = -1;
    if (hipDeviceSynchronize() != hipSuccess) {
        *err = -1;
        delete c;
        return nullptr;
    }
    // the no-allocation ladder's scratch address on this device, taken now, outside any capture (a failure here is
    // retried by that entry point's first call)
    (void)pch::noalloc_prepare();
    return c;
}

void pcx_ctx_free(pcx_ctx* c) {
    if (!c) return;
    for (hipEvent_t e : c->ev) (void)hipEventDestroy(e);
    delete c;
}

int pcx_timing(pcx_ctx* c, int max_stages) {
    if (!c || max_stages < 0) return -1;
    if (max_stages == 0) {
        c->timing = false;
        return 0;
    }
    while (c->ev.size() < 2 * (size_t)max_stages) {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) return -1;
        c->ev.push_back(e);
    }
    c->ev_stage.assign(c->ev.size() / 2, -1);
    c->ev_used = 0;
    c->timing = true;
    return 0;
}

int pcx_timing_read(pcx_ctx* c, int stage, double* total_ms, int* count) {
    if (!c || !total_ms || !count) return -1;
    double t = 0;
    int n = 0;
    for (size_t i = 0; i < c->ev_used; ++i) {
        if (c->ev_stage[i] != stage) continue;
        float ms = 0;
        hipError_t e = hipEventElapsedTime(&ms, c->ev[2 * i], c->ev[2 * i + 1]);
        if (e != hipSuccess) return (int)e;
        t += ms;
        ++n;
    }
    *total_ms = t;
    *count = n;
    return 0;
}
const KernelTable* pcx_ctx_table(const pcx_ctx* c) { return c->tab; }
const PrimeConst* pcx_ctx_primes(const pcx_ctx* c) { return c->pr; }
const void* pcx_ctx_twiddle(const pcx_ctx* c, int which) {
    switch (which) {
        case 0: return c->fw;
        case 1: return c->fws;
        case 2: return c->iw;
        case 3: return c->iws;
        case 4: return c->ninv;
        case 5: return c->ninvs;
        default: return nullptr;
    }
}
uint64_t pcx_ctx_root(const pcx_ctx* c, int id) { return id >= 0 && id < c->rows ? c->roots[id] : 0; }
size_t pcx_ctx_workspace_bytes(const pcx_ctx* c) { return c->ws_bytes; }

int pcx_ctx_table_only(pcx_ctx* c, int on) {
    if (!c) return -1;
    const int prev = c->table_only;
    c->table_only = on ? 1 : 0;
    c->md_fused = on ? 0 : c->md_fused_init;
    return prev;
}
int pcx_ctx_conv_fusion(pcx_ctx* c, int mask) {
    if (!c) return -1;
    const int prev = c->cc_fused;
    if (mask >= 0) c->cc_fused = mask & 7;
    return prev;
}
size_t pcx_ct_words(const pcx_ctx* c) { return c->ct_words(); }

pcx_rows* pcx_rows_new(pcx_ctx* c, const uint32_t* roff, const int32_t* ids, int nrows) {
    if (nrows < 0) return nullptr;
    for (int i = 0; i < nrows; ++i)
        if (ids[i] < 0 || ids[i] >= c->rows) return nullptr;
    pcx_rows* r = new (std::nothrow) pcx_rows;
    if (!r) return nullptr;
    // prime-major (a stable sort by prime id): the rows are independent, and neighbouring workgroups then read one
    // prime's twiddle tables from L2 instead of each row's from further out
    std::vector<int> ord(nrows);
    for (int i = 0; i < nrows; ++i) ord[i] = i;
    std::stable_sort(ord.begin(), ord.end(), [&](int a, int b) { return ids[a] < ids[b]; });
    std::vector<uint32_t> ro(nrows);
    std::vector<int32_t> rp(nrows);
    for (int i = 0; i < nrows; ++i) {
        ro[i] = roff[ord[i]];
        rp[i] = ids[ord[i]];
    }
    if (fill_rows(r->dev, r->r, ro, rp, nullptr, nullptr)) {
        delete r;
        return nullptr;
    }
    return r;
}
void pcx_rows_free(pcx_rows* r) { delete r; }

int pcx_ntt_one_pass_min(int rows) { return pch::ntt_one_pass_min(rows); }

int pcx_ntt(pcx_ctx* c, int dir, void* base, const pcx_rows* rows, pc_stream_t s) {
    if (!c || !rows || (dir != 1 && dir != -1)) return -1;
    NttArgs a = ntt_args(c, base, rows->r, rows->r.n);
    return dir == 1 ? c->tab->ntt_fwd(&a, s) : c->tab->ntt_inv(&a, s);
}

// A key group from host b ([ndig][srows][N] per key, dense words) and seeds, banded at q_top (nq - 1: full rows)
static pcx_keys* keys_new(pcx_ctx* c, int nkeys, const uint64_t* galois, const uint32_t* seeds,
                          const uint32_t* const* b_host, int bits, int q_top, int* err) {
    int dummy;
    if (!err) err = &dummy;
    *err = 0;
    if (!c || !galois || !seeds || !b_host || q_top < 0 || q_top >= c->nq) {
        *err = -1;
        return nullptr;
    }
    pcx_keys* k = keys_shell(c, nkeys, galois, bits, err);
    if (!k) return nullptr;
    if (q_top < c->nq - 1) {
        // crates/pc-gpu/src/keys.rs:86-92 KskShape::banded: every digit whose first prime is <= q_top
        k->q_top = q_top;
        k->ndig = q_top / c->alpha + 1;
        k->srows = q_top + 1 + c->kp;
    }
    const uint32_t n = c->n;
    const size_t nrow = (size_t)k->ndig * k->srows;
    std::vector<const void*> kb;
    std::vector<const uint32_t*> sd;
    for (int r = 0; r < nkeys; ++r) {
        std::vector<uint32_t> s(seeds + 8 * r, seeds + 8 * r + 8);
        sd.push_back(k->dev.upload(s));
        std::vector<uint32_t> st;
        if (bits == 0) {
            st.assign(b_host[r], b_host[r] + nrow * n);
        } else {
            st.assign(nrow * k->row_words, 0);
            for (size_t q = 0; q < nrow; ++q) pack_row(b_host[r] + q * n, n, bits, &st[q * k->row_words], k->row_words);
        }
        void* p = k->dev.upload(st);
        k->b_ptr.push_back(p);
        kb.push_back(p);
    }
    k->kb = (const void**)k->dev.upload(kb);
    k->seed = (const uint32_t**)k->dev.upload(sd);
    k->seed_ptr = sd;
    if (!k->dev.err && k->q_top < 0) {
        // the retry-value table is indexed by prime id: full-layout groups only (a band redraws in the dot)
        if (int e = build_patches(c, k)) k->dev.err = e;
    }
    if (k->dev.err) {
        *err = k->dev.err;
        delete k;
        return nullptr;
    }
    return k;
}

pcx_keys* pcx_keys_new(pcx_ctx* c, int nkeys, const uint64_t* galois, const uint32_t* seeds,
                       const uint32_t* const* b_host, int bits, int* err) {
    return keys_new(c, nkeys, galois, seeds, b_host, bits, c ? c->nq - 1 : 0, err);
}
pcx_keys* pcx_keys_new_banded(pcx_ctx* c, int nkeys, const uint64_t* galois, const uint32_t* seeds,
                              const uint32_t* const* b_host, int bits, int q_top, int* err) {
    return keys_new(c, nkeys, galois, seeds, b_host, bits, q_top, err);
}
int pcx_keys_q_top(const pcx_keys* k) { return k ? (k->q_top < 0 ? k->c->nq - 1 : k->q_top) : -1; }

// crates/pc-gpu/src/keygen.rs:172-262: the secret's eval rows, per key the Gaussian errors NTT'd, s_new =
// sigma_{g^-1}(s) by the automorph kernel, then ksk_gen (b dense or packed); sq: the old secret squared in the kernel
// (the relinearization key s^2 -> s, galois 1; keygen.rs:225-226)
static pcx_keys* keys_generate(pcx_ctx* c, int nkeys, const uint64_t* galois, const int8_t* secret, const uint32_t* seeds,
                        const int64_t* errors, int bits, int sq, int* err) {
    int dummy;
    if (!err) err = &dummy;
    *err = 0;
    pcx_keys* k = keys_shell(c, nkeys, galois, bits, err);
    if (!k) return nullptr;
    const uint32_t n = c->n;
    const int R = c->rows;
    hipStream_t s = nullptr;
    // secret eval rows [R][N]
    std::vector<uint32_t> sh((size_t)R * n);
    for (int t = 0; t < R; ++t) {
        const uint32_t p = (uint32_t)c->primes[t];
        for (uint32_t i = 0; i < n; ++i) sh[(size_t)t * n + i] = secret[i] >= 0 ? (uint32_t)secret[i] : p - (uint32_t)(-secret[i]);
    }
    Dev tmp;
    uint32_t* s_eval = tmp.upload(sh);
    uint32_t* s_new = (uint32_t*)tmp.alloc((size_t)R * n * 4);
    uint32_t* e = (uint32_t*)tmp.alloc((size_t)c->dnum * R * n * 4);
    std::vector<uint32_t> all_roff, e_roff;
    std::vector<int32_t> all_ids, e_ids;
    for (int t = 0; t < R; ++t) all_roff.push_back(t), all_ids.push_back(t);
    for (int d = 0; d < c->dnum; ++d)
        for (int t = 0; t < R; ++t) e_roff.push_back(d * R + t), e_ids.push_back(t);
    std::vector<int32_t> ids(all_ids);
    Rows rows_all, rows_e;
    fill_rows(tmp, rows_all, all_roff, all_ids, nullptr, nullptr);
    fill_rows(tmp, rows_e, e_roff, e_ids, nullptr, nullptr);
    int32_t* d_ids = tmp.upload(ids);
    if (tmp.err) {
        *err = tmp.err;
        delete k;
        return nullptr;
    }
    NttArgs a = ntt_args(c, s_eval, rows_all, R);
    int rc = c->tab->ntt_fwd(&a, s);
    std::vector<const void*> kb;
    std::vector<const uint32_t*> sd;
    for (int r = 0; r < nkeys && !rc; ++r) {
        std::vector<uint32_t> sv(seeds + 8 * r, seeds + 8 * r + 8);
        uint32_t* dseed = k->dev.upload(sv);
        sd.push_back(dseed);
        // errors: e_d mod q_t for every row of digit d
        std::vector<uint32_t> eh((size_t)c->dnum * R * n);
        for (int d = 0; d < c->dnum; ++d)
            for (int t = 0; t < R; ++t) {
                const int64_t p = (int64_t)c->primes[t];
                const int64_t* ev = errors + ((size_t)r * c->dnum + d) * n;
                uint32_t* o = &eh[((size_t)d * R + t) * n];
                for (uint32_t i = 0; i < n; ++i) o[i] = (uint32_t)(((ev[i] % p) + p) % p);
            }
        if (hipMemcpy(e, eh.data(), eh.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
            rc = -1;
            break;
        }
        NttArgs ea = ntt_args(c, e, rows_e, c->dnum * R);
        if ((rc = c->tab->ntt_fwd(&ea, s))) break;
        AutomorphArgs au;
        memset(&au, 0, sizeof au);
        au.out = PolyRef{s_new, 0, 0};
        au.in = PolyRef{s_eval, 0, 0};
        au.rs = RowSet{R, 0, 0, 0};
        au.pr = c->pr;
        au.k = k->autok_h[r];
        au.K = 1;
        au.nparts = 1;
        if ((rc = c->tab->automorph(&au, s))) break;
        const uint64_t words = (uint64_t)c->dnum * R * k->row_words;
        void* b = k->dev.alloc(words * 4);
        if (!b) {
            rc = -1;
            break;
        }
        k->b_ptr.push_back(b);
        kb.push_back(b);
        KskGenArgs g;
        memset(&g, 0, sizeof g);
        g.b = b;
        g.a = nullptr;
        g.e = e;
        g.s_new = s_new;
        g.s_old = s_eval;
        g.seed = dseed;
        g.ids = d_ids;
        g.digit_of = c->digit_of;
        g.pmod = c->pmod;
        g.pmods = c->pmod + R;
        g.pr = c->pr;
        g.row_words = k->row_words;
        g.nrows = R;
        g.ndig = c->dnum;
        g.nq = c->nq;
        g.bits = bits;
        g.sq = sq;
        if ((rc = c->tab->ksk_gen(&g, s))) break;
        if (hipDeviceSynchronize() != hipSuccess) rc = -1;
    }
    if (!rc) {
        k->kb = (const void**)k->dev.upload(kb);
        k->seed = (const uint32_t**)k->dev.upload(sd);
        k->seed_ptr = sd;
        if (k->dev.err) rc = k->dev.err;
    }
    if (!rc) rc = build_patches(c, k);
    if (!rc && hipDeviceSynchronize() != hipSuccess) rc = -1;
    if (rc) {
        *err = rc;
        delete k;
        return nullptr;
    }
    return k;
}

pcx_keys* pcx_keys_generate(pcx_ctx* c, int nkeys, const uint64_t* galois, const int8_t* secret,
                            const uint32_t* seeds, const int64_t* errors, int bits, int* err) {
    return keys_generate(c, nkeys, galois, secret, seeds, errors, bits, 0, err);
}

pcx_keys* pcx_keys_relin(pcx_ctx* c, const int8_t* secret, const uint32_t* seed, const int64_t* errors, int bits,
                         int* err) {
    const uint64_t one = 1;
    return keys_generate(c, 1, &one, secret, seed, errors, bits, 1, err);
}

void pcx_keys_free(pcx_keys* k) { delete k; }

size_t pcx_keys_patch_bytes(const pcx_keys* k) { return k ? k->patch_words * 4 : 0; }

int pcx_keys_resident_a(pcx_keys* k, int regen_digits, pc_stream_t s) {
    if (!k || regen_digits < 0 || k->q_top >= 0 || (int)k->seed_ptr.size() != k->nkeys) return -1;
    pcx_ctx* c = k->c;
    if (!k->ka && regen_digits < c->dnum) {
        // every key's a expanded once: [dnum][rows][N] words, prime-id rows (the table's ksk_expand)
        std::vector<int32_t> ids(c->rows);
        for (int i = 0; i < c->rows; ++i) ids[i] = i;
        const int32_t* dids = k->dev.upload(ids);
        std::vector<const void*> ka;
        for (int r = 0; r < k->nkeys && !k->dev.err; ++r) {
            void* p = k->dev.alloc((size_t)c->dnum * c->rows * c->n * 4);
            if (!p) break;
            KskExpandArgs e;
            memset(&e, 0, sizeof e);
            e.out = p;
            e.seed = k->seed_ptr[r];
            e.prime_ids = dids;
            e.pr = c->pr;
            e.nmod = c->rows;
            e.dnum = c->dnum;
            e.d0 = 0;
            if (int rc = c->tab->ksk_expand(&e, s)) return rc;
            ka.push_back(p);
        }
        if (k->dev.err) return k->dev.err;
        k->ka = (const void**)k->dev.upload(ka);
        if (!k->ka) return k->dev.err ? k->dev.err : -1;
        if (int rc = pc_hip_stream_sync(s)) return rc;
    }
    k->regen = regen_digits;
    return 0;
}
size_t pcx_keys_resident_bytes(const pcx_keys* k) {
    return k && k->ka ? (size_t)k->nkeys * k->c->dnum * k->c->rows * k->c->n * 4 : 0;
}

int pcx_keys_download_b(pcx_keys* k, int r, uint32_t* b_host) {
    if (!k || r < 0 || r >= k->nkeys) return -1;
    pcx_ctx* c = k->c;
    const size_t nrow = (size_t)k->ndig * k->srows;
    std::vector<uint32_t> st(nrow * k->row_words);
    if (hipMemcpy(st.data(), k->b_ptr[r], st.size() * 4, hipMemcpyDeviceToHost) != hipSuccess) return -1;
    for (size_t q = 0; q < nrow; ++q) {
        const uint32_t* w = &st[q * k->row_words];
        uint32_t* o = b_host + q * c->n;
        if (k->bits == 0) {
            memcpy(o, w, (size_t)c->n * 4);
            continue;
        }
        const uint32_t mask = k->bits == 32 ? 0xFFFFFFFFu : (1u << k->bits) - 1u;
        for (uint32_t i = 0; i < c->n; ++i) {
            const uint64_t bit = (uint64_t)i * k->bits;
            const uint64_t v = ((uint64_t)w[(bit >> 5) + 1] << 32 | w[bit >> 5]) >> (bit & 31);
            o[i] = (uint32_t)v & mask;
        }
    }
    return 0;
}

int pcx_modup(pcx_ctx* c, const void* ct, int top, pc_stream_t s) { return modup(c, ct, top, s); }
const void* pcx_modup_digits(const pcx_ctx* c) { return c->digits; }
int pcx_dot(pcx_ctx* c, pcx_keys* k, int r, const void* ct, int top, void* ext, pc_stream_t s) {
    return dot(c, k, r, 1, ct, top, ext, s);
}
int pcx_moddown(pcx_ctx* c, void* ext, int top, void* out, pc_stream_t s) {
    return c ? moddown(c, ext, c->conv, 1, top, out, s) : -1;
}

int pcx_rotate(pcx_ctx* c, pcx_keys* k, int r, const void* ct, int top, void* out, pc_stream_t s) {
    if (!c || !k || r < 0 || r >= k->nkeys || !level(c, top) || !serves(k, top)) return -1;
    if (k->galois[r] == 1) return copy_q(c, ct, top, out, s);
    if (int e = modup(c, ct, top, s)) return e;
    if (int e = dot(c, k, r, 1, ct, top, c->ext, s)) return e;
    return moddown(c, c->ext, c->conv, 1, top, out, s);
}

int pcx_cts_stage_hoisted(pcx_ctx* c, pcx_keys* k, int r0, int B, int G, const void* const* pts, int npts, int ptw,
                          uint32_t enc, const void* ct, int top, void* rot, void* res, pc_stream_t s) {
    const Level* L = c ? level(c, top) : nullptr;
    if (!L || !k || k->c != c || B < 1 || G < 1 || npts < 0 || !pts || !ct || !rot || !res) return -1;
    if (!serves(k, top)) return -1;
    if (B > 1 && (r0 < 0 || r0 + B - 1 > k->nkeys)) return -1;
    const uint64_t part = (uint64_t)c->rows * c->n;
    // rot_0 = P ct on Q rows 0..top, zero on the special rows
    EwArgs e;
    memset(&e, 0, sizeof e);
    e.out = PolyRef{rot, 2 * part, part};
    e.a = PolyRef{const_cast<void*>(ct), 2 * part, part};
    e.rs = RowSet{top + 1, c->kp, c->nq, 0};
    e.sc = c->pmod;
    e.scs = c->pmod + (c->nq + c->kp);
    e.pr = c->pr;
    e.K = 1;
    e.nparts = 2;
    e.zero_p = 1;
    if (int er = c->tab->ew_scale(&e, s)) return er;
    // rot_i (i >= 1): the babies' key switches before ModDown, one ModUp and one dot launch for the B - 1 keys
    if (B > 1) {
        if (int er = modup(c, ct, top, s)) return er;
        if (int er = dot(c, k, r0, B - 1, ct, top, (uint32_t*)rot + c->ct_words(), s)) return er;
    }
    PtDotArgs a;
    memset(&a, 0, sizeof a);
    a.rot = PolyRef{rot, (uint64_t)B * c->ct_words(), part};
    a.res = PolyRef{res, (uint64_t)G * c->ct_words(), part};
    a.rot_stride = c->ct_words();
    a.res_stride = c->ct_words();
    a.pts = pts;
    a.pr = c->pr;
    a.rs = RowSet{top + 1, c->kp, c->nq, 0};
    a.npts = npts;
    a.bstep = B;
    a.gstep = G;
    a.K = 1;
    a.ptw = ptw;
    a.pt_prow = top + 1;
    a.enc = enc;
    Stage st(c, 7, s);
    return c->tab->pt_dot(&a, s);
}

int pcx_moddown_k(pcx_ctx* c, void* ext, int top, void* out, int m, pc_stream_t s) {
    if (!c || !ext || !out || m < 1 || m > c->k_rot || !level(c, top)) return -1;
    return moddown(c, ext, c->conv, m, top, out, s);
}

int pcx_cts_stage(pcx_ctx* c, pcx_keys* k, int r0, int B, int G, const void* const* pts, int npts, int ptw,
                  uint32_t enc, const void* ct, int top, void* res, pc_stream_t s) {
    const Level* L = c ? level(c, top) : nullptr;
    if (!L || !k || k->c != c || B < 1 || G < 1 || npts < 0 || !pts || !ct || !res) return -1;
    if (!serves(k, top)) return -1;
    if (B > 1 && (r0 < 0 || r0 + B - 1 > k->nkeys)) return -1;
    if (B > 1)
        if (int e = modup(c, ct, top, s)) return e;
    CtsRegenArgs ra;
    memset(&ra, 0, sizeof ra);
    CtsArgs& a = ra.cts;
    a.x = ct;
    a.modup = c->digits;
    a.kinv = k->kinv + (B > 1 ? r0 : 0);
    a.rows = L->ks_rows;
    a.digit_of = c->digit_of;
    a.pmod = c->pmod;
    a.pmods = c->pmod + (c->nq + c->kp);
    a.pr = c->pr;
    a.ct_stride = c->ct_words();
    a.part_stride = (uint64_t)c->rows * c->n;
    a.mu_ct_stride = (uint64_t)c->dnum * c->rows * c->n;
    a.mu_digit_stride = (uint64_t)c->rows * c->n;
    a.K = 1;
    a.B = B;
    a.ndig = L->ndig;
    a.nq = c->nq;
    a.nlive = top + 1;
    a.ptw = ptw;
    a.pt_prow = top + 1;
    a.enc = enc;
    a.nrows = L->nks;
    a.kmax = 1;
    a.pair_cts = 2;  // giant steps 2l, 2l + 1 at res + 2l, 2l + 1 cts: the results contiguous
    KeyTab& t = ra.key;
    t.kb = k->kb + (B > 1 ? r0 : 0);
    t.seed = k->seed + (B > 1 ? r0 : 0);
    t.row_words = k->row_words;
    t.bits = k->bits;
    t.q_top = k->q_top;
    t.srows = k->srows;
    t.nregen = k->ndig;
    Stage st(c, 7, s);
    for (int j0 = 0; j0 < G; j0 += 4) {
        // up to four giant steps per launch: the baby keys regenerated once per launch
        a.G = std::min(4, G - j0);
        a.pts = pts + (size_t)j0 * B;
        a.npts = std::max(0, npts - j0 * B);
        a.res = (uint32_t*)res + (size_t)j0 * c->ct_words();
        if (int e = c->tab->cts_fused_regen(&ra, s)) return e;
    }
    return 0;
}

int pcx_rotate_hoisted(pcx_ctx* c, pcx_keys* k, const int* idx, int n, const void* ct, int top, void* out,
                       pc_stream_t s) {
    if (!c || !k || n < 1 || !level(c, top) || !serves(k, top)) return -1;
    for (int j = 0; j < n; ++j)
        if (idx[j] < 0 || idx[j] >= k->nkeys) return -1;
    const size_t cw = c->ct_words();
    bool live = false;
    for (int j = 0; j < n; ++j) {
        if (k->galois[idx[j]] == 1) {
            if (int e = copy_q(c, ct, top, (uint32_t*)out + j * cw, s)) return e;
        } else {
            live = true;
        }
    }
    if (!live) return 0;
    if (int e = modup(c, ct, top, s)) return e;
    int j = 0;
    while (j < n) {
        if (k->galois[idx[j]] == 1) {
            ++j;
            continue;
        }
        // a chunk: consecutive outputs whose keys are consecutive in the group (one dot launch)
        int m = 1;
        while (j + m < n && m < c->k_rot && idx[j + m] == idx[j] + m && k->galois[idx[j + m]] != 1) ++m;
        if (int e = dot(c, k, idx[j], m, ct, top, c->ext, s)) return e;
        if (int e = moddown(c, c->ext, c->conv, m, top, (uint32_t*)out + j * cw, s)) return e;
        j += m;
    }
    return 0;
}

int pcx_rotate_sum(pcx_ctx* c, pcx_keys* k, const int* idx, int n, const void* ct, int top, void* out,
                   const void* onto, pc_stream_t s) {
    if (!c || !k || k->c != c || n < 1 || !idx || !ct || !out || !level(c, top) || !serves(k, top)) return -1;
    for (int j = 0; j < n; ++j)
        if (idx[j] < 0 || idx[j] >= k->nkeys || k->galois[idx[j]] == 1) return -1;  // no step 0 in a sum group
    if (int e = modup(c, ct, top, s)) return e;
    // runs of consecutive keys, one summed dot each, the later runs added onto the first's sum
    for (int j = 0; j < n;) {
        int m = 1;
        while (j + m < n && idx[j + m] == idx[j] + m) ++m;
        if (int e = dot(c, k, idx[j], m, ct, top, c->ext, s, j == 0 ? 1 : 2)) return e;
        j += m;
    }
    return moddown(c, c->ext, c->conv, 1, top, out, s, onto);
}

// the extended sum of pcx_rotate_many in c->ext: one ModUp per input (each its own c1), c0 folded in as P sigma(c0).
// When every run's keys are consecutive and the n dots fit c->ext: each run's dots as one diagonal launch, input j's
// into extended slot j (*nsum = n: the ModDown reads their sum); else each dot written (the first) or added onto one
// sum (*nsum = 1).
static int rotate_many_ext(pcx_ctx* c, pcx_keys* k, const int* idx, int n, const void* const* cts, int top,
                           pc_stream_t s, int* nsum) {
    if (!c || !k || k->c != c || n < 1 || !idx || !cts || !level(c, top) || !serves(k, top)) return -1;
    for (int j = 0; j < n; ++j)
        if (!cts[j] || idx[j] < 0 || idx[j] >= k->nkeys || k->galois[idx[j]] == 1) return -1;
    // runs of up to k_max inputs laid out ct_words apart share one ModUp launch sequence; each input's dot then reads
    // its own digits
    const size_t cw = c->ct_words(), dw = (size_t)c->dnum * c->rows * c->n;
    bool diag = n > 1 && n <= std::max(c->k_rot, c->k_max) && k->pval && !c->table_only;
    for (int j0 = 0, m = 1; j0 < n && diag; j0 += m, m = 1) {
        while (j0 + m < n && m < c->k_max && cts[j0 + m] == (const void*)((const uint32_t*)cts[j0] + m * cw)) ++m;
        for (int j = j0 + 1; j < j0 + m; ++j) diag = diag && idx[j] == idx[j0] + (j - j0);
    }
    *nsum = 1;
    for (int j0 = 0; j0 < n;) {
        int m = 1;
        while (j0 + m < n && m < c->k_max && cts[j0 + m] == (const void*)((const uint32_t*)cts[j0] + m * cw)) ++m;
        if (int e = modup(c, cts[j0], top, s, m)) return e;
        if (diag) {
            const int e = dot_diag(c, k, idx[j0], m, cts[j0], top, c->ext + (size_t)j0 * cw, c->digits, s);
            if (e == 0) {
                *nsum = j0 + m;
                j0 += m;
                continue;
            }
            if (e != -2 || j0 > 0) return e;
            diag = false;  // the diagonal form does not apply: every dot onto one sum
        }
        for (int j = j0; j < j0 + m; ++j)
            if (int e = dot(c, k, idx[j], 1, cts[j], top, c->ext, s, 0, j ? 1 | PC_KS_ACC : 1, 1,
                            c->digits + (size_t)(j - j0) * dw))
                return e;
        j0 += m;
    }
    return 0;
}

int pcx_rotate_many(pcx_ctx* c, pcx_keys* k, const int* idx, int n, const void* const* cts, int top, void* out,
                    const void* onto, pc_stream_t s) {
    if (!out) return -1;
    int nsum = 1;
    if (int e = rotate_many_ext(c, k, idx, n, cts, top, s, &nsum)) return e;
    return moddown(c, c->ext, c->conv, 1, top, out, s, onto, nsum);
}

int pcx_rotate_many_rescale(pcx_ctx* c, pcx_keys* k, const int* idx, int n, const void* const* cts, int top,
                            void* out, const void* onto, pc_stream_t s) {
    if (!out || top < 2) return -1;
    int nsum = 1;
    if (int e = rotate_many_ext(c, k, idx, n, cts, top, s, &nsum)) return e;
    return moddown_rescale(c, c->ext, top, out, onto, s, 1, nsum);
}

// pcx_rotate_sum over K <= min(k_max, k_rot) consecutive ciphertexts: one ModUp launch sequence for the K, each
// ciphertext's summed key dots into its own extended slot (reading its own digits), one ModDown of the K onto onto
static int rotate_sum_k(pcx_ctx* c, pcx_keys* k, const int* idx, int n, const void* ct, int K, int top, void* out,
                        const void* onto, pc_stream_t s) {
    if (K < 1 || K > c->k_max || K > c->k_rot) return -1;
    for (int j = 0; j < n; ++j)
        if (idx[j] < 0 || idx[j] >= k->nkeys || k->galois[idx[j]] == 1) return -1;
    const size_t cw = c->ct_words(), dw = (size_t)c->dnum * c->rows * c->n;
    if (int e = modup(c, ct, top, s, K)) return e;
    // runs of consecutive keys, each one summed dot over up to 4 of the ciphertexts at a time
    for (int j = 0; j < n;) {
        int m = 1;
        while (j + m < n && idx[j + m] == idx[j] + m) ++m;
        for (int k0 = 0; k0 < K; k0 += 4) {
            const int kc = std::min(4, K - k0);
            if (int e = dot(c, k, idx[j], m, (const uint32_t*)ct + k0 * cw, top, c->ext + k0 * cw, s, j == 0 ? 1 : 2, 1,
                            kc, c->digits + k0 * dw))
                return e;
        }
        j += m;
    }
    return moddown(c, c->ext, c->conv, K, top, out, s, onto);
}

int pcx_rotate_and_sum_k(pcx_ctx* c, pcx_keys* k, const void* x, int top, int64_t start, int64_t stop,
                         int radix_bits, void* out, void* tmp, int K, pc_stream_t s) {
    if (!c || !k || k->c != c || !x || !out || !tmp || !level(c, top) || K < 1 || !serves(k, top)) return -1;
    const size_t cw = c->ct_words();
    if (K == 1) return pcx_rotate_and_sum(c, k, x, top, start, stop, radix_bits, out, tmp, s);
    if (start == 0 || stop <= 0 || K > c->k_max || K > c->k_rot) return -1;
    const uint64_t m2 = 2ull * c->n;
    auto key_of = [&](int64_t st) {
        const int64_t h = (int64_t)(c->n / 2);
        const uint64_t r = (uint64_t)(((st % h) + h) % h);
        const uint64_t g = powmod(5, r, m2);
        for (int i = 0; i < k->nkeys; ++i)
            if (k->galois[i] == g) return i;
        return -1;
    };
    const int64_t sign = start > 0 ? 1 : -1, gap = start > 0 ? start : -start;
    if (gap >= stop) return copy_q(c, x, top, out, s, K);
    int64_t gaps[64];
    size_t ng = 0;
    for (int64_t g = gap; g < stop && ng < 64; g *= 2) gaps[ng++] = g;
    // every rung a radix rung of at most 8 bits whose steps the group holds: the K ciphertexts go rung by rung
    // together; otherwise each takes the one-ciphertext ladder
    const size_t rb = radix_bits >= 2 ? (size_t)radix_bits : 1;
    bool batched = rb >= 2 && rb <= 8;
    int keys[64][255];
    int cnts[64];
    size_t nr = 0;
    for (size_t i0 = 0; batched && i0 < ng; ++nr) {
        const size_t n = std::min(rb, ng - i0);
        cnts[nr] = (int)(((int64_t)1 << n) - 1);
        for (int j = 1; j <= cnts[nr] && batched; ++j) batched = (keys[nr][j - 1] = key_of(sign * j * gaps[i0])) >= 0;
        batched = batched && n > 1;
        i0 += n;
    }
    if (!batched) {
        for (int kk = 0; kk < K; ++kk)
            if (int e = pcx_rotate_and_sum(c, k, (const uint32_t*)x + kk * cw, top, start, stop, radix_bits,
                                           (uint32_t*)out + kk * cw, (uint32_t*)tmp + kk * cw, s))
                return e;
        return 0;
    }
    if (x != out)
        if (int e = copy_q(c, x, top, out, s, K)) return e;
    for (size_t r = 0; r < nr; ++r)
        if (int e = rotate_sum_k(c, k, keys[r], cnts[r], out, K, top, out, out, s)) return e;
    return 0;
}

int pcx_rotate_and_sum(pcx_ctx* c, pcx_keys* k, const void* x, int top, int64_t start, int64_t stop, int radix_bits,
                       void* out, void* tmp, pc_stream_t s) {
    if (!c || !k || k->c != c || !x || !out || !tmp || !level(c, top) || !serves(k, top)) return -1;
    if (start == 0 || stop <= 0) return -1;
    const uint64_t m2 = 2ull * c->n;
    // the key of a rotation step (g = 5^step mod 2N; negative steps by the inverse), -1 if the group has none
    auto key_of = [&](int64_t st) {
        const int64_t h = (int64_t)(c->n / 2);
        const uint64_t r = (uint64_t)(((st % h) + h) % h);
        const uint64_t g = powmod(5, r, m2);
        for (int i = 0; i < k->nkeys; ++i)
            if (k->galois[i] == g) return i;
        return -1;
    };
    const int64_t sign = start > 0 ? 1 : -1, gap = start > 0 ? start : -start;
    if (gap >= stop) return copy_q(c, x, top, out, s);
    // the rungs' gaps (doubling from |start| below stop: at most 63) and, for rungs of up to 8 bits, their key lists in
    // fixed arrays: the ladder itself allocates nothing on the host or the device
    int64_t gaps[64];
    size_t ng = 0;
    for (int64_t g = gap; g < stop && ng < 64; g *= 2) gaps[ng++] = g;
    const size_t rb = radix_bits >= 2 ? (size_t)radix_bits : 1;
    bool have = false;
    for (size_t i0 = 0; i0 < ng;) {
        const size_t n = std::min(rb, ng - i0);
        if (rb >= 2 && n > 1) {
            // one rung of radix 2^n: out += sum over j < 2^n of rot(out, j gap) when the group holds every step
            int small[255];
            std::vector<int> big;
            const int64_t cnt = ((int64_t)1 << n) - 1;
            if (n > 8) big.resize((size_t)cnt);
            int* idx = n > 8 ? big.data() : small;
            bool all = true;
            for (int64_t j = 1; j <= cnt; ++j) all = (idx[j - 1] = key_of(sign * j * gaps[i0])) >= 0 && all;
            if (all) {
                if (!have) {
                    if (int e = copy_q(c, x, top, out, s)) return e;
                    have = true;
                }
                if (int e = pcx_rotate_sum(c, k, idx, (int)cnt, out, top, out, out, s)) return e;
                i0 += n;
                continue;
            }
        }
        for (size_t r = 0; r < n; ++r) {
            const int key = key_of(sign * gaps[i0 + r]);
            if (key < 0) return -1;
            // tmp = rot(out, step) (rot(x, step) on the first rung), then out += tmp
            if (int e = pcx_rotate(c, k, key, have ? out : x, top, tmp, s)) return e;
            if (!have) {
                if (int e = copy_q(c, x, top, out, s)) return e;
                have = true;
            }
            if (int e = add_q(c, out, tmp, top, out, s)) return e;
        }
        i0 += n;
    }
    return 0;
}


// Rescale by the top ndrop (1 or 2) primes (crates/pc-gpu/src/rescale.rs:318-440): out's rows 0..top - ndrop become
// the rescale of ct's rows 0..top (both parts, eval form); out's rows above are left as scratch. Two primes: INTT of
// the tops, rescale_fwd (the corrections generated in the forward NTT's column pass, out = alpha out + NTT(tmp) in its
// epilogue); one prime: INTT of the top, rescale_coef, the NTT of the corrections with the same epilogue.
int pcx_rescale_k(pcx_ctx* c, const void* ct, int top, int ndrop, void* out, int K, pc_stream_t s) {
    if (!c || !ct || !out || (ndrop != 1 && ndrop != 2) || top < ndrop || top >= c->nq || K < 1 || K > c->k_max)
        return -1;
    const Level::Rescale& Z = c->levels[top].rs[ndrop - 1];
    const int R = c->rows;
    Stage st(c, 9, s);
    if (ct != out)
        if (int e = copy_q(c, ct, top, out, s, K)) return e;
    NttArgs in = ntt_args(c, out, Z.intt, k_rows(c, Z.intt, K));
    if (int e = c->tab->ntt_inv(&in, s)) return e;
    RescaleArgs r;
    memset(&r, 0, sizeof r);
    const uint64_t part = (uint64_t)R * c->n;
    r.x = PolyRef{out, 2 * part, part};
    r.tmp = PolyRef{c->tmp, 2 * part, part};
    r.A = Z.k;
    r.As = Z.k + R;
    r.B = Z.k + 2 * R;
    r.Bs = Z.k + 3 * R;
    r.qam = Z.k + 6 * R;
    r.qbm = Z.k + 7 * R;
    r.pr = c->pr;
    r.qinv_ab = Z.qinv_ab;
    r.C_ab = Z.C_ab;
    r.ca = r.cb = 1;
    r.top = top;
    r.nrows = top + 1 - ndrop;
    r.K = K;
    r.ndrop = ndrop;
    NttArgs f = ntt_args(c, c->tmp, Z.ntt, k_rows(c, Z.ntt, K));
    f.epi = 3;
    f.eout = out;
    f.ex = out;
    f.xnum = 1;
    f.es = Z.k + 4 * R;
    f.ess = Z.k + 5 * R;
    if (ndrop == 2) {
        RescaleNttArgs a;
        a.rs = r;
        a.ntt = f;
        return c->tab->rescale_fwd(&a, s);
    }
    if (int e = c->tab->rescale_coef(&r, s)) return e;
    return c->tab->ntt_fwd(&f, s);
}
int pcx_rescale(pcx_ctx* c, const void* ct, int top, int ndrop, void* out, pc_stream_t s) {
    return pcx_rescale_k(c, ct, top, ndrop, out, 1, s);
}

// The relinearized product (crates/pc-gpu/src/relin.rs:213-235 mult, Cached-key form :119-128): (c0, c1, d2) by the
// tensor kernel (d2 into part 1 of the context's tmp ciphertext), ModUp(d2), the key inner product with the
// relinearization key (no c0 term, no automorphism), and the ModDown added onto (c0, c1): out = (c0, c1) +
// (ext - conv) P^-1 on Q rows 0..top. out may be a or b.
// the product's (d0, d1) into out and the key switch of d2 into c->ext (before ModDown)
// The tensor (d0, d1 into out, d2 into c->tmp), d2's ModUp and its key dot into c->ext. *folded: the dot also added
// P (d0, d1) on the Q rows (the fast dot's c0 mode 3), so the ModDown has nothing to add onto; else out keeps (d0, d1)
// for the ModDown's add-onto step.
static int relin_ext(pcx_ctx* c, pcx_keys* k, const void* a, const void* b, int top, void* out, pc_stream_t s,
                     bool* folded, int K = 1, int twice = 0) {
    if (!c || !k || !a || !b || !out || top < 0 || top >= c->nq || k->nkeys < 1 || k->galois[0] != 1) return -1;
    if (K < 1 || K > c->k_max || K > 4 || !serves(k, top)) return -1;  // the key dot takes at most 4 ciphertexts
    const uint64_t part = (uint64_t)c->rows * c->n;
    TensorArgs t;
    memset(&t, 0, sizeof t);
    t.out = PolyRef{out, 2 * part, part};
    t.d2 = PolyRef{c->tmp, 2 * part, part};
    t.a0 = t.a1 = PolyRef{const_cast<void*>(a), 2 * part, part};
    t.b0 = t.b1 = PolyRef{const_cast<void*>(b), 2 * part, part};
    t.pr = c->pr;
    t.npairs = 1;
    t.n = top + 1;
    t.K = K;
    t.dbl = twice ? 1 : 0;  // 2 (a b): the same residues as the product of 2a and b
    {
        Stage st(c, 8, s);
        if (int e = c->tab->tensor(&t, s)) return e;
    }
    if (int e = modup(c, c->tmp, top, s, K)) return e;
    // the fast dot with the retry table takes (d0, d1) as its c0 mode 3
    const Level* L = level(c, top);
    *folded = k->pval && !c->table_only && k->bits == 0 && L->ndig >= 1 && L->ndig <= 3;
    return dot(c, k, 0, 1, c->tmp, top, c->ext, s, 0, *folded ? 3 : 0, K, nullptr, *folded ? out : nullptr);
}
int pcx_mul_relin(pcx_ctx* c, pcx_keys* k, const void* a, const void* b, int top, void* out, pc_stream_t s) {
    bool folded = false;
    if (int e = relin_ext(c, k, a, b, top, out, s, &folded)) return e;
    return moddown(c, c->ext, c->conv, 1, top, out, s, folded ? nullptr : out);
}
int pcx_mul_relin_rescale(pcx_ctx* c, pcx_keys* k, const void* a, const void* b, int top, void* out,
                          pc_stream_t s) {
    return pcx_mul_relin_rescale_k(c, k, a, b, top, out, 1, 0, s);
}
int pcx_mul_relin_rescale_k(pcx_ctx* c, pcx_keys* k, const void* a, const void* b, int top, void* out, int K,
                            int twice, pc_stream_t s) {
    if (top < 2) return -1;
    bool folded = false;
    if (int e = relin_ext(c, k, a, b, top, out, s, &folded, K, twice)) return e;
    return moddown_rescale(c, c->ext, top, out, folded ? nullptr : out, s, K);
}

int pcx_mul_relin_rescale_list(pcx_ctx* c, pcx_keys* k, const void* const* a, const void* const* b, int K, int top,
                               void* out, int twice, pc_stream_t s) {
    if (!c || !k || !a || !b || !out || top < 2 || top >= c->nq || k->nkeys < 1 || k->galois[0] != 1) return -1;
    if (K < 1 || K > c->k_max || K > pch::TLIST_MAX || !serves(k, top)) return -1;
    const uint64_t part = (uint64_t)c->rows * c->n;
    pch::TensorListArgs t;
    memset(&t, 0, sizeof t);
    // out slot i may be an operand of pair i itself (the tensor reads each word before storing it, in one thread),
    // but must not overlap any other pair's operands: the launch stores slot i while other workgroups read them
    const uintptr_t cwb = (uintptr_t)c->ct_words() * sizeof(uint32_t);
    for (int j = 0; j < K; ++j) {
        if (!a[j] || !b[j]) return -1;
        t.a[j] = (const uint32_t*)a[j];
        t.b[j] = (const uint32_t*)b[j];
        for (int i = 0; i < K; ++i) {
            const uintptr_t o = (uintptr_t)out + i * cwb;
            for (const void* x : {a[j], b[j]}) {
                const uintptr_t xv = (uintptr_t)x;
                if (xv < o + cwb && o < xv + cwb && !(i == j && xv == o)) return -1;
            }
        }
    }
    t.out = (uint32_t*)out;
    t.d2 = c->tmp;
    t.part = part;
    t.ct_stride = 2 * part;
    t.pr = c->pr;
    t.n = top + 1;
    t.K = K;
    t.dbl = twice ? 1 : 0;
    {
        Stage st(c, 8, s);
        if (int e = pch::tensor_list((int)c->logn, &t, s)) return e;
    }
    if (int e = modup(c, c->tmp, top, s, K)) return e;
    // the key dots four ciphertexts at a time, (d0, d1) folded in as in relin_ext
    const Level* L = level(c, top);
    const bool folded = k->pval && !c->table_only && k->bits == 0 && L->ndig >= 1 && L->ndig <= 3;
    const size_t cw = c->ct_words(), dw = (size_t)c->dnum * c->rows * c->n;
    for (int j0 = 0; j0 < K; j0 += 4) {
        const int m = std::min(4, K - j0);
        if (int e = dot(c, k, 0, 1, c->tmp + j0 * cw, top, c->ext + j0 * cw, s, 0, folded ? 3 : 0, m,
                        c->digits + j0 * dw, folded ? (const uint32_t*)out + j0 * cw : nullptr))
            return e;
    }
    return moddown_rescale(c, c->ext, top, out, folded ? nullptr : out, s, K);
}

int pcx_mul_sum_relin_rescale_list(pcx_ctx* c, pcx_keys* k, const void* const* a, const void* const* b,
                                   const int* off, int K, int top, const void* const* y, const void* const* yk,
                                   unsigned ysub, int twice, void* out, pc_stream_t s) {
    if (!c || !k || !a || !b || !off || !out || top < 2 || top >= c->nq || k->nkeys < 1 || k->galois[0] != 1) return -1;
    if (K < 1 || K > c->k_max || !serves(k, top) || off[0] != 0) return -1;
    for (int j = 0; j < K; ++j)
        if (off[j + 1] <= off[j] || off[j + 1] > pch::TLIST_MAX) return -1;
    const uint64_t part = (uint64_t)c->rows * c->n;
    pch::TensorListArgs t;
    memset(&t, 0, sizeof t);
    // no out slot may overlap any operand: the one tensor launch stores every slot while it reads every pair
    const uintptr_t cwb = (uintptr_t)c->ct_words() * sizeof(uint32_t);
    for (int j = 0; j < off[K]; ++j) {
        if (!a[j] || !b[j]) return -1;
        t.a[j] = (const uint32_t*)a[j];
        t.b[j] = (const uint32_t*)b[j];
        for (const void* x : {a[j], b[j]}) {
            const uintptr_t xv = (uintptr_t)x, o = (uintptr_t)out;
            if (xv < o + K * cwb && o < xv + cwb) return -1;
        }
    }
    for (int j = 0; y && j < K; ++j) {
        if (!y[j]) continue;
        const uintptr_t yv = (uintptr_t)y[j], o = (uintptr_t)out;
        if (yv < o + K * cwb && o < yv + cwb) return -1;
        t.y[j] = (const uint32_t*)y[j];
        t.yk[j] = yk ? (const uint32_t*)yk[j] : nullptr;
        t.ysub |= ((ysub >> j) & 1u) << j;
    }
    t.krows = c->rows;
    t.dbl = twice ? 1 : 0;
    t.sum = 1;
    for (int j = 0; j <= K; ++j) t.off[j] = off[j];
    t.out = (uint32_t*)out;
    t.d2 = c->tmp;
    t.part = part;
    t.ct_stride = 2 * part;
    t.pr = c->pr;
    t.n = top + 1;
    t.K = K;
    {
        Stage st(c, 8, s);
        if (int e = pch::tensor_list((int)c->logn, &t, s)) return e;
    }
    if (int e = modup(c, c->tmp, top, s, K)) return e;
    const Level* L = level(c, top);
    const bool folded = k->pval && !c->table_only && k->bits == 0 && L->ndig >= 1 && L->ndig <= 3;
    const size_t cw = c->ct_words(), dw = (size_t)c->dnum * c->rows * c->n;
    for (int j0 = 0; j0 < K; j0 += 4) {
        const int m = std::min(4, K - j0);
        if (int e = dot(c, k, 0, 1, c->tmp + j0 * cw, top, c->ext + j0 * cw, s, 0, folded ? 3 : 0, m,
                        c->digits + j0 * dw, folded ? (const uint32_t*)out + j0 * cw : nullptr))
            return e;
    }
    return moddown_rescale(c, c->ext, top, out, folded ? nullptr : out, s, K);
}

int pcx_mul_plain_k(pcx_ctx* c, const void* ct, const void* const* pts, int K, int top, void* out, pc_stream_t s) {
    if (!c || !ct || !pts || !out || top < 0 || top >= c->nq || K < 1 || K > pch::TLIST_MAX) return -1;
    pch::MulPtListArgs m;
    memset(&m, 0, sizeof m);
    for (int j = 0; j < K; ++j) {
        if (!pts[j]) return -1;
        m.t[j] = (const uint32_t*)pts[j];
    }
    m.in = (const uint32_t*)ct;
    m.out = (uint32_t*)out;
    m.part = (uint64_t)c->rows * c->n;
    m.ct_stride = c->ct_words();
    m.pr = c->pr;
    m.n = top + 1;
    m.K = K;
    return pch::mul_pt_list((int)c->logn, &m, s);
}

// The plaintext product (crates/pc-gpu/src/ops.rs:927-951 mult_pt, the table's mul_table, em.cuh:508-515): out = ct pt
// on Q rows 0..top of both parts, pt one plaintext of evaluation-form rows by prime id. out may be ct.
int pcx_mul_plain(pcx_ctx* c, const void* ct, const void* pt, int top, void* out, pc_stream_t s) {
    if (!c || !ct || !pt || !out || top < 0 || top >= c->nq) return -1;
    const uint64_t part = (uint64_t)c->rows * c->n;
    MulTableArgs m;
    memset(&m, 0, sizeof m);
    m.out = PolyRef{out, 2 * part, part};
    m.in = PolyRef{const_cast<void*>(ct), 2 * part, part};
    m.t = pt;
    m.pr = c->pr;
    m.n = top + 1;
    m.K = 1;
    return c->tab->mul_table(&m, s);
}

// Decryption on the device (crates/pc-gpu/src/decrypt.rs:27-117 Decryptor): c0 + c1 s over the bottom d rows of each
// ciphertext through the tensor kernel with the key pair (s, 1) (its middle term x0 c1 + x1 c0; the other two terms
// land in part 0 and are discarded), then the inverse NTT of those rows. Its own buffers: the key pairs
// [which][part][d][N] and k_max outputs [c][part][d][N]; the INTT row lists for 1..k_max ciphertexts.
struct pcx_decryptor {
    pcx_ctx* c = nullptr;
    int d = 0, k_max = 0;
    int loaded[2] = {0, 0};
    Dev dev;
    uint32_t *key = nullptr, *out = nullptr;
    std::vector<Rows> lists;
};

pcx_decryptor* pcx_decryptor_new(pcx_ctx* c, int d, int k_max, int* err) {
    auto fail = [&](int e) -> pcx_decryptor* {
        if (err) *err = e;
        return nullptr;
    };
    if (!c || d < 1 || d > c->nq || k_max < 1) return fail(-1);
    pcx_decryptor* x = new (std::nothrow) pcx_decryptor;
    if (!x) return fail(-1);
    x->c = c;
    x->d = d;
    x->k_max = k_max;
    const size_t n = c->n;
    x->key = (uint32_t*)x->dev.alloc(4 * d * n * sizeof(uint32_t));
    x->out = (uint32_t*)x->dev.alloc((size_t)k_max * 2 * d * n * sizeof(uint32_t));
    x->lists.resize(k_max);
    for (int k = 1; k <= k_max && !x->dev.err; ++k) {
        std::vector<uint32_t> ro;
        std::vector<int32_t> rp;
        for (int r = 0; r < d; ++r)  // prime-major
            for (int cc = 0; cc < k; ++cc) {
                ro.push_back((uint32_t)(cc * 2 * d + d + r));
                rp.push_back(r);
            }
        if (fill_rows(x->dev, x->lists[k - 1], ro, rp, nullptr, nullptr)) break;
    }
    if (x->dev.err || !x->key || !x->out) {
        const int e = x->dev.err ? x->dev.err : -1;
        delete x;
        return fail(e);
    }
    if (err) *err = 0;
    return x;
}
void pcx_decryptor_free(pcx_decryptor* x) { delete x; }

// The secret's evaluation-form rows 0..d-1 ([nwhich][d][N], host): dense, then sparse when nwhich is 2
// (decrypt.rs:65-77 load_secret). Synchronises s.
int pcx_decryptor_load_secret(pcx_decryptor* x, const uint32_t* s_rows, int nwhich, pc_stream_t s) {
    if (!x || !s_rows || nwhich < 1 || nwhich > 2) return -1;
    const size_t n = x->c->n, dn = (size_t)x->d * n;
    std::vector<uint32_t> host(4 * dn, 0);
    for (int w = 0; w < nwhich; ++w) {
        for (int r = 0; r < x->d; ++r)
            for (size_t i = 0; i < n; ++i)
                if (s_rows[w * dn + r * n + i] >= x->c->primes[r]) return -1;
        memcpy(&host[w * 2 * dn], s_rows + w * dn, dn * sizeof(uint32_t));
        std::fill(host.begin() + w * 2 * dn + dn, host.begin() + (w + 1) * 2 * dn, 1u);
    }
    hipError_t e = hipMemcpyAsync(x->key, host.data(), host.size() * sizeof(uint32_t), hipMemcpyHostToDevice,
                                  (hipStream_t)s);
    if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)s);
    if (e != hipSuccess) return (int)e;
    x->loaded[0] = 1;
    x->loaded[1] = nwhich == 2;
    return 0;
}

// Coefficient rows of c0 + c1 s on rows 0..d-1 of K ciphertexts (ct: K consecutive ciphertexts of the context's
// layout, top >= d - 1) into out [K][d][N] (device), enqueued on s (decrypt.rs:79-117 decrypt_rows, without its
// download: the caller reads out). which: 0 dense secret, 1 sparse.
int pcx_decrypt_rows(pcx_decryptor* x, const void* ct, int K, int top, int which, void* out, pc_stream_t s) {
    if (!x || !ct || !out || K < 1 || K > x->k_max || which < 0 || which > 1 || !x->loaded[which]) return -1;
    pcx_ctx* c = x->c;
    if (top < x->d - 1 || top >= c->nq) return -1;
    const uint64_t n = c->n, dn = (uint64_t)x->d * n, part = (uint64_t)c->rows * n;
    TensorArgs t;
    memset(&t, 0, sizeof t);
    t.out = PolyRef{x->out, 2 * dn, dn};
    t.d2 = PolyRef{x->out, 2 * dn, 0};  // part 1 of d2 is part 0 of out
    t.a0 = PolyRef{x->key + which * 2 * dn, 0, dn};
    t.b0 = PolyRef{const_cast<void*>(ct), 2 * part, part};
    t.pr = c->pr;
    t.npairs = 1;
    t.n = x->d;
    t.K = K;
    if (int e = c->tab->tensor(&t, s)) return e;
    const Rows& r = x->lists[K - 1];
    NttArgs a = ntt_args(c, x->out, r, r.n);
    if (int e = c->tab->ntt_inv(&a, s)) return e;
    for (int cc = 0; cc < K; ++cc) {
        hipError_t e = hipMemcpyAsync((uint32_t*)out + cc * dn, x->out + cc * 2 * dn + dn, dn * sizeof(uint32_t),
                                      hipMemcpyDeviceToDevice, (hipStream_t)s);
        if (e != hipSuccess) return (int)e;
    }
    return 0;
}

}  // extern "C"
