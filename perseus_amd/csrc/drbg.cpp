// The key-generation sampler on the host: the DRBG, the sparse ternary secret, the discrete Gaussian and the draw order
// of a switching key's seed and errors (crates/pc-core/src/keys.rs:113-325 Prng, sample_sparse_ternary,
// DiscreteGaussian; crates/pc-gpu/src/keygen.rs:193-210 generate_with's host draws). The device side of key
// generation (pcx_keys_generate: the errors' NTT, the automorphism of the secret, the key rows) takes these errors.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <new>
#include <vector>

#include "pc_hip.h"

namespace {

constexpr uint32_t DRBG_WORD = 0x47425244u;  // "DRBG": state word 15 of every block

inline uint32_t rol(uint32_t x, int r) { return (x << r) | (x >> (32 - r)); }

// ChaCha20: the constants, the 8 key words, then state words 12..15 as given; 10 double rounds and the feed-forward
void block20(const uint32_t key[8], uint32_t w12, uint32_t w13, uint32_t w14, uint32_t w15, uint32_t out[16]) {
    uint32_t s[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u, key[0], key[1], key[2], key[3],
                      key[4],      key[5],      key[6],      key[7],      w12,    w13,    w14,    w15};
    uint32_t x[16];
    memcpy(x, s, sizeof x);
    auto q = [&x](int a, int b, int c, int d) {
        x[a] += x[b], x[d] = rol(x[d] ^ x[a], 16);
        x[c] += x[d], x[b] = rol(x[b] ^ x[c], 12);
        x[a] += x[b], x[d] = rol(x[d] ^ x[a], 8);
        x[c] += x[d], x[b] = rol(x[b] ^ x[c], 7);
    };
    for (int r = 0; r < 10; ++r) {
        q(0, 4, 8, 12), q(1, 5, 9, 13), q(2, 6, 10, 14), q(3, 7, 11, 15);
        q(0, 5, 10, 15), q(1, 6, 11, 12), q(2, 7, 8, 13), q(3, 4, 9, 14);
    }
    for (int i = 0; i < 16; ++i) out[i] = x[i] + s[i];
}

// cdf[k] = P(|X| <= k) of the discrete Gaussian of width sigma on |x| <= ceil(14 sigma): weights exp(-k^2 / 2 sigma^2)
// (doubled for k > 0), normalised by their sum taken in order, accumulated in order
std::vector<double> gauss_cdf(double sigma) {
    const size_t bound = (size_t)ceil(sigma * 14.0);
    std::vector<double> w(bound + 1), cdf(bound + 1);
    double tot = 0.0;
    for (size_t k = 0; k <= bound; ++k) {
        const double e = exp(-((double)(k * k)) / (2.0 * sigma * sigma));
        w[k] = k == 0 ? e : 2.0 * e;
        tot += w[k];
    }
    double acc = 0.0;
    for (size_t k = 0; k <= bound; ++k) {
        acc += w[k] / tot;
        cdf[k] = acc;
    }
    return cdf;
}

}  // namespace

struct pcx_drbg {
    uint32_t key[8];
    uint32_t stream;
    uint64_t ctr = 0;
    uint32_t buf[16];
    int used = 16;
    uint32_t u32() {
        if (used == 16) {
            block20(key, (uint32_t)ctr, (uint32_t)(ctr >> 32), stream, DRBG_WORD, buf);
            ++ctr;
            used = 0;
        }
        return buf[used++];
    }
    uint64_t u64() {
        const uint64_t lo = u32();
        return lo | (uint64_t)u32() << 32;
    }
    // uniform in [0, q): words below 2^64 mod q are rejected, so the accepted range is a multiple of q
    uint64_t below(uint64_t q) {
        const uint64_t rej = (UINT64_MAX % q + 1) % q;
        for (;;) {
            const uint64_t v = u64();
            if (v >= rej) return v % q;
        }
    }
    double f64() { return (double)(u64() >> 11) * (1.0 / 9007199254740992.0); }
    void gaussian(const std::vector<double>& cdf, uint32_t n, int64_t* out) {
        for (uint32_t i = 0; i < n; ++i) {
            const double u = f64();
            const size_t k = std::min<size_t>(std::upper_bound(cdf.begin(), cdf.end(), u) - cdf.begin(), cdf.size() - 1);
            out[i] = k == 0 ? 0 : (u32() & 1) == 0 ? (int64_t)k : -(int64_t)k;
        }
    }
};

extern "C" {
pcx_drbg* pcx_drbg_new(const uint32_t key[8], uint32_t stream) {
    if (!key) return nullptr;
    pcx_drbg* g = new (std::nothrow) pcx_drbg;
    if (!g) return nullptr;
    memcpy(g->key, key, sizeof g->key);
    g->stream = stream;
    return g;
}
void pcx_drbg_free(pcx_drbg* g) { delete g; }
uint32_t pcx_drbg_u32(pcx_drbg* g) { return g ? g->u32() : 0; }
int pcx_drbg_ksk_seed(pcx_drbg* g, uint32_t out[8]) {
    if (!g || !out) return -1;
    for (int i = 0; i < 8; ++i) out[i] = g->u32();
    return 0;
}
int pcx_drbg_sparse_ternary(pcx_drbg* g, uint32_t n, uint32_t h, int8_t* out) {
    if (!g || !out || h > n) return -1;
    memset(out, 0, n);
    for (uint32_t placed = 0; placed < h;) {
        const uint64_t i = g->below(n);
        if (out[i] == 0) {
            out[i] = (g->u32() & 1) == 0 ? 1 : -1;
            ++placed;
        }
    }
    return 0;
}
int pcx_drbg_gaussian(pcx_drbg* g, double sigma, uint32_t n, int64_t* out) {
    if (!g || !out || !(sigma > 0.0 && sigma < 1e6)) return -1;
    g->gaussian(gauss_cdf(sigma), n, out);
    return 0;
}
int pcx_keygen_draw(pcx_drbg* g, int nkeys, int ndig, uint32_t n, double sigma, uint32_t* seeds, int64_t* errors) {
    if (!g || nkeys < 0 || ndig < 1 || !seeds || !errors || !(sigma > 0.0 && sigma < 1e6)) return -1;
    const std::vector<double> cdf = gauss_cdf(sigma);
    for (int r = 0; r < nkeys; ++r) {
        uint32_t sub[8];
        pcx_drbg_ksk_seed(g, seeds + 8 * (size_t)r);
        pcx_drbg_ksk_seed(g, sub);
        for (int d = 0; d < ndig; ++d) {
            pcx_drbg e;
            memcpy(e.key, sub, sizeof sub);
            e.stream = (uint32_t)d;
            e.gaussian(cdf, n, errors + ((size_t)r * ndig + d) * n);
        }
    }
    return 0;
}
}
