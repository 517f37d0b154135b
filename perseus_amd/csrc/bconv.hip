// Batched fast base conversion (crates/pc-kernels/kernels/args.cuh:109-141; host twin crates/pc-host/src/bconv.rs):
//   y_i = x_i pre_i mod s_i (prescaled jobs: y_i = x_i as stored), out_t = sum_i y_i M[i][t] mod t;
//   exact jobs: v = sum_i y_i rb_i (double FMA in source order), u = floor(v + 0.5) (centred: the lift's mean),
//   out_t -= u (B mod t).
// One launch for every job of a plan: grid (N / (256 V), njobs, target groups), 256 threads of V consecutive
// coefficients (V = 1); the job's targets are split over up to ceil(max_tgt / TPG) groups (each re-reads the job's
// sources, from L2), so that a few wide jobs still put several waves on every SIMD.
//
// 31-bit primes break the reference's lazy bound nsrc (p - 1)^2 < 2^64 past 4 sources, so the sum of products is
// carried in 96 bits (a 64-bit sum and a count of its wraps) and reduced once: the exact integer formula, whatever
// the width of the primes.
#include "common.h"

namespace pch {
namespace bconv {

constexpr int BX = 256;
constexpr int MAX_REG_SRC = 20;  // the fused ModDown-rescale's kp + 2 sources at 16 special primes
constexpr int TPG = 8;  // targets per workgroup when BconvArgs.max_tgt gives the grid its target groups

struct Pool {
    const uint32_t* w;
    int ns, nt;
    __device__ uint32_t src_row(int i) const { return w[i]; }
    __device__ uint32_t src_prime(int i) const { return w[ns + i]; }
    __device__ uint32_t pre(int i) const { return w[2 * ns + i]; }
    __device__ uint32_t tgt_row(int t) const { return w[3 * ns + t]; }
    __device__ uint32_t tgt_prime(int t) const { return w[3 * ns + nt + t]; }
    __device__ uint32_t m(int i, int t) const { return w[3 * ns + 2 * nt + i * nt + t]; }
};

// the exact jobs' tables after M (build_tables, crates/pc-gpu/src/bconv.rs:94-121): rb[ns] doubles at the first
// 8-byte aligned word, then bmod[nt]
__device__ __forceinline__ const double* exact_rb(const uint32_t* pool_base, const BconvJob& j) {
    size_t w = (size_t)j.pool_off + 3 * j.nsrc + 2 * j.ntgt + (size_t)j.nsrc * j.ntgt;
    if (w & 1) ++w;  // the pool is 8-byte aligned: word parity is byte alignment
    return (const double*)(pool_base + w);
}

__device__ __forceinline__ uint64_t exact_u(const BconvJob& j, const double* rb, const uint32_t* y, int stride,
                                            uint32_t coef) {
    if (j.exact == 2) {
        // the mean-centred job (crates/pc-host/src/bconv.rs:70-76): ns / 2, odd ns rounded by a hash of the index
        const uint64_t ns = j.nsrc;
        return (ns >> 1) + ((ns & 1) & ((coef * 0x9E3779B1u) >> 31));
    }
    double v = 0.0;
    for (uint32_t i = 0; i < j.nsrc; ++i) v = __fma_rn((double)y[i * stride], rb[i], v);
    return (uint64_t)floor(v + 0.5);
}

// One workgroup = one job x 256 V coefficients (V per thread). A job's record lives in device memory, so its size is
// read here: jobs of at most 20 sources keep the sources of their V coefficients in registers and the job's tables in
// LDS; wider jobs (bconv_wide, up to 48 sources at u32 words) re-read their sources per target (L1/L2 resident).
__device__ __forceinline__ void job_wide(const BconvArgs& A, const BconvJob& j, const Pool& P, const uint32_t* src,
                                         uint32_t* dst, uint32_t c, int logn, int t0, int t1) {
    auto yv = [&](int i) {
        uint32_t v = src[((size_t)P.src_row(i) << logn) + c];
        if (!j.prescaled) v = Red(A.pr[P.src_prime(i)]).mul(v, P.pre(i));
        return v;
    };
    uint64_t u = 0;
    const uint32_t* bmod = nullptr;
    if (j.exact) {
        const double* rb = exact_rb((const uint32_t*)A.pool, j);
        bmod = (const uint32_t*)(rb + j.nsrc);
        if (j.exact == 2) {
            const uint64_t ns = j.nsrc;
            u = (ns >> 1) + ((ns & 1) & ((c * 0x9E3779B1u) >> 31));
        } else {
            double v = 0.0;
            for (int i = 0; i < P.ns; ++i) v = __fma_rn((double)yv(i), rb[i], v);
            u = (uint64_t)floor(v + 0.5);
        }
    }
    for (int t = t0; t < t1; ++t) {
        const Red red(A.pr[P.tgt_prime(t)]);
        uint64_t acc = 0;
        uint32_t wraps = 0;
        // groups of four products (below 2^64 for words below 2^31), one carry per group
        for (int i = 0; i < P.ns; i += 4) {
            uint64_t cs = 0;
            for (int e = i; e < i + 4 && e < P.ns; ++e) cs += (uint64_t)yv(e) * P.m(e, t);
            acc += cs;
            wraps += acc < cs;
        }
        uint32_t r = red.red96(acc, wraps);
        if (j.exact) r = subm(r, red((uint64_t)u * bmod[t]), red.p);
        dst[((size_t)P.tgt_row(t) << logn) + c] = r;
    }
}

// The job's tables in LDS (jobs of at most 20 sources and MAXT targets): M transposed and zero-padded to 20 sources,
// so a target's column is broadcast 16-byte reads; each target's reduction constants; the sources' rows and pre.
constexpr int MAXT = 64;
struct JobLds {
    uint32_t mt[MAXT][MAX_REG_SRC];
    uint32_t trow[MAXT];
    uint32_t tc[MAXT][4];  // p, 2^32 mod p, its Shoup companion, floor(2^32 / p)
    uint32_t r64[MAXT];    // 2^64 mod p
    uint32_t r64k[MAXT][8];  // k 2^64 mod p, k < 8 (the wraps of a 96-bit sum of at most 20 products)
    double rb[MAX_REG_SRC];
    uint32_t bmod[MAXT][2];  // B mod p and its Shoup companion
    uint32_t sp[MAX_REG_SRC];  // the sources' primes
};

// V consecutive words at p (V = 2 or 4: one 8- or 16-byte access)
template <int V>
__device__ __forceinline__ void ldv(const uint32_t* p, uint32_t (&v)[V]) {
    if constexpr (V == 1) {
        v[0] = *p;
    } else if constexpr (V == 4) {
        const uint4 x = *(const uint4*)p;
        v[0] = x.x, v[1] = x.y, v[2] = x.z, v[3] = x.w;
    } else {
        const uint2 x = *(const uint2*)p;
        v[0] = x.x, v[1] = x.y;
    }
}
template <int V>
__device__ __forceinline__ void stv(uint32_t* p, const uint32_t (&v)[V]) {
    if constexpr (V == 1) *p = v[0];
    else if constexpr (V == 4) *(uint4*)p = make_uint4(v[0], v[1], v[2], v[3]);
    else *(uint2*)p = make_uint2(v[0], v[1]);
}

// the V source words of each source at c0, as stored (zero past the job's sources)
template <int V>
__device__ __forceinline__ void load_sources(const Pool& P, const uint32_t* src, uint32_t c0, int logn,
                                             uint32_t (&y)[MAX_REG_SRC * V]) {
#pragma unroll
    for (int i = 0; i < MAX_REG_SRC; ++i) {
        uint32_t v[V] = {};
        if (i < P.ns) ldv<V>(src + ((size_t)P.src_row(i) << logn) + c0, v);
#pragma unroll
        for (int k = 0; k < V; ++k) y[i * V + k] = v[k];
    }
}

template <int V>
__device__ __forceinline__ void job_lds(const BconvArgs& A, const BconvJob& j, const Pool& P, const JobLds& S,
                                        uint32_t (&y)[MAX_REG_SRC * V], uint32_t* dst, uint32_t c0, int logn, int ntl) {
    if (!j.prescaled) {
#pragma unroll
        for (int i = 0; i < MAX_REG_SRC; ++i) {
            if (i < P.ns) {
                const Red red(A.pr[P.src_prime(i)]);
                const uint32_t pre = P.pre(i);
#pragma unroll
                for (int k = 0; k < V; ++k) y[i * V + k] = red.mul(y[i * V + k], pre);
            }
        }
    }
    // sources are reduced below their prime, M's entries below the target's: ns products of at most
    // (max source prime - 1) (p_t - 1) each
    uint32_t mx = 0;
    for (int i = 0; i < P.ns; ++i) mx = max(mx, S.sp[i]);
    const uint64_t lazy_bound = ~0ull / (uint64_t)P.ns;
    uint64_t u[V] = {};
    if (j.exact) {
#pragma unroll
        for (int k = 0; k < V; ++k) {
            if (j.exact == 2) {
                const uint64_t ns = j.nsrc;
                u[k] = (ns >> 1) + ((ns & 1) & (((c0 + k) * 0x9E3779B1u) >> 31));
            } else {
                double v = 0.0;
#pragma unroll
                for (int i = 0; i < MAX_REG_SRC; ++i)
                    if (i < P.ns) v = __fma_rn((double)y[i * V + k], S.rb[i], v);
                u[k] = (uint64_t)floor(v + 0.5);
            }
        }
    }
    const int ng = (P.ns + 3) >> 2;  // groups of 4 sources (M zero-padded)
    for (int t = 0; t < ntl; ++t) {
        const Red red(S.tc[t][0], S.tc[t][1], S.tc[t][2], S.tc[t][3]);
        const uint32_t r64 = S.r64[t];
        const uint64_t pm = (uint64_t)(mx - 1) * (uint64_t)(red.p - 1);  // the largest product
        uint64_t acc[V] = {};
        uint32_t r[V];
        if (pm <= lazy_bound) {
            // every partial sum stays below 2^64: one multiply-add per product
#pragma unroll
            for (int g = 0; g < MAX_REG_SRC / 4; ++g) {
                if (g < ng) {
                    const uint4 m4 = *(const uint4*)&S.mt[t][4 * g];
                    const uint32_t mv[4] = {m4.x, m4.y, m4.z, m4.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
#pragma unroll
                        for (int k = 0; k < V; ++k) acc[k] += (uint64_t)y[(4 * g + e) * V + k] * mv[e];
                    }
                }
            }
#pragma unroll
            for (int k = 0; k < V; ++k) r[k] = red(acc[k]);
        } else if (pm <= ~0ull / 16) {
            // 16 products fit a 64-bit sum (30-bit primes): sources 0..15 in one, the rest in a second; their sum's
            // carry is folded in as 2^64 mod p
            uint64_t acc2[V] = {};
#pragma unroll
            for (int g = 0; g < MAX_REG_SRC / 4; ++g) {
                if (g < ng) {
                    const uint4 m4 = *(const uint4*)&S.mt[t][4 * g];
                    const uint32_t mv[4] = {m4.x, m4.y, m4.z, m4.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
#pragma unroll
                        for (int k = 0; k < V; ++k) {
                            const uint64_t pr = (uint64_t)y[(4 * g + e) * V + k] * mv[e];
                            if (g < 4) acc[k] += pr;
                            else acc2[k] += pr;
                        }
                    }
                }
            }
#pragma unroll
            for (int k = 0; k < V; ++k) {
                const uint64_t s2 = acc[k] + acc2[k];
                r[k] = addm(red(s2), s2 < acc[k] ? r64 : 0u, red.p);
            }
        } else {
            // four products of words below 2^31 stay below 2^64: each group of four (the last one as long as the
            // sources go) is summed by multiply-adds, and only the group sums carry into the 96-bit total; its at most
            // 4 wraps come back as wraps 2^64 mod p from the table
            uint32_t wraps[V] = {};
#pragma unroll
            for (int g = 0; g < MAX_REG_SRC / 4; ++g) {
                if (g < ng) {
                    const uint4 m4 = *(const uint4*)&S.mt[t][4 * g];
                    const uint32_t mv[4] = {m4.x, m4.y, m4.z, m4.w};
                    uint64_t cs[V] = {};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if (4 * g + e < P.ns) {
#pragma unroll
                            for (int k = 0; k < V; ++k) cs[k] += (uint64_t)y[(4 * g + e) * V + k] * mv[e];
                        }
                    }
#pragma unroll
                    for (int k = 0; k < V; ++k) {
                        if (g == 0) {
                            acc[k] = cs[k];
                        } else {
                            acc[k] += cs[k];
                            wraps[k] += acc[k] < cs[k];
                        }
                    }
                }
            }
#pragma unroll
            for (int k = 0; k < V; ++k) r[k] = addm(red(acc[k]), S.r64k[t][wraps[k]], red.p);
        }
        // exact jobs: u <= nsrc, so u B mod p is one Shoup product
#pragma unroll
        for (int k = 0; k < V; ++k) {
            if (j.exact) r[k] = subm(r[k], shoup((uint32_t)u[k], S.bmod[t][0], S.bmod[t][1], red.p), red.p);
        }
        stv<V>(dst + ((size_t)S.trow[t] << logn) + c0, r);
    }
}

template <int V>
__global__ void __launch_bounds__(BX) bconv_k(BconvArgs A, int logn) {
    __shared__ JobLds S;
    const BconvJob j = A.jobs[blockIdx.y];
    const Pool P{(const uint32_t*)A.pool + j.pool_off, (int)j.nsrc, (int)j.ntgt};
    const uint32_t c0 = blockIdx.x * (BX * V) + threadIdx.x * V;
    if (P.ns < 1) return;
    // this workgroup's targets [t0, t0 + ntl): the job's targets split evenly over the grid's target groups
    const int tpg = (P.nt + (int)gridDim.z - 1) / (int)gridDim.z;
    const int t0 = (int)blockIdx.z * tpg;
    const int ntl = P.nt - t0 < tpg ? P.nt - t0 : tpg;
    if (ntl <= 0) return;
    const uint32_t* src = (const uint32_t*)A.src + ((size_t)j.src_off << logn);
    uint32_t* dst = (uint32_t*)A.dst + ((size_t)j.dst_off << logn);
    if (P.ns <= MAX_REG_SRC && ntl <= MAXT) {
        // the sources' loads first: their round trips (row ids, then words) overlap the tables' (ids, then primes)
        uint32_t y[MAX_REG_SRC * V];
        if (c0 < (1u << logn)) load_sources<V>(P, src, c0, logn, y);
        for (int e = threadIdx.x; e < ntl * MAX_REG_SRC; e += BX) {
            const int t = e / MAX_REG_SRC, i = e % MAX_REG_SRC;
            S.mt[t][i] = (t < ntl && i < P.ns) ? P.m(i, t0 + t) : 0;
        }
        // every table load of the set-up is issued by its own thread: one round trip to the pool, one to the primes
        if (threadIdx.x < P.ns) S.sp[threadIdx.x] = (uint32_t)A.pr[P.src_prime(threadIdx.x)].p;
        for (int t = threadIdx.x; t < ntl; t += BX) {
            const PrimeConst& q = A.pr[P.tgt_prime(t0 + t)];
            S.trow[t] = P.tgt_row(t0 + t);
            const uint32_t qp = (uint32_t)q.p, r32 = (uint32_t)q.split, r32s = (uint32_t)(q.split >> 32);
            S.tc[t][0] = qp;
            S.tc[t][1] = r32;
            S.tc[t][2] = r32s;
            S.tc[t][3] = (uint32_t)(q.mu_lo >> 32);
            const uint32_t r64 = shoup(r32, r32, r32s, qp);
            S.r64[t] = r64;
            uint32_t v = 0;
            for (int k = 0; k < 8; ++k, v = addm(v, r64, qp)) S.r64k[t][k] = v;
        }
        if (j.exact) {
            const double* rb = exact_rb((const uint32_t*)A.pool, j);
            const uint32_t* bmod = (const uint32_t*)(rb + j.nsrc);
            for (int i = threadIdx.x; i < P.ns; i += BX) S.rb[i] = rb[i];
            for (int t = threadIdx.x; t < ntl; t += BX) {
                const uint32_t b = bmod[t0 + t], qp = (uint32_t)A.pr[P.tgt_prime(t0 + t)].p;
                S.bmod[t][0] = b;
                S.bmod[t][1] = (uint32_t)(((uint64_t)b << 32) / qp);
            }
        }
        __syncthreads();
        if (c0 < (1u << logn)) job_lds<V>(A, j, P, S, y, dst, c0, logn, ntl);
    } else if (c0 < (1u << logn)) {
        for (int k = 0; k < V; ++k) job_wide(A, j, P, src, dst, c0 + k, logn, t0, t0 + ntl);
    }
}

inline int check(const BconvArgs* a) {
    if (!a || !a->src || !a->dst || !a->jobs || !a->pool || !a->pr || a->njobs < 0) return -1;
    return 0;
}

template <int LOGN>
int launch(const BconvArgs* a, pc_stream_t s) {
    if (int rc = check(a)) return rc;
    if (a->njobs == 0) return 0;
    // target groups: every job's targets fit max_tgt (the plan's widest job; 0: one group). Each group re-reads the
    // job's sources, so a launch splits its targets only as far as it needs workgroups: about 2048 in all, with at
    // least TPG targets per group (a ModDown of 7 ciphertexts takes 2 groups instead of 6). One coefficient per thread
    // measured best on the bootstrap (14.97 ms against 15.25 at two, same box; 4 coefficients, 4 or 16 to 64 targets
    // per group and 4096 workgroups were no better) and equal on the C3 batch.
    constexpr int V = 1;
    const int gx = ((1 << LOGN) + BX * V - 1) / (BX * V);
    const int gmax = a->max_tgt > TPG ? std::min((a->max_tgt + TPG - 1) / TPG, 256) : 1;
    const long base = (long)gx * a->njobs;
    const int gz = (int)std::max(1L, std::min((long)gmax, (2048 + base - 1) / base));
    hipLaunchKernelGGL(bconv_k<V>, dim3(gx, a->njobs, gz), dim3(BX), 0, (hipStream_t)s, *a, LOGN);
    return launch_rc();
}

}  // namespace bconv
}  // namespace pch

namespace pch {
#define PCH_BCONV_INST(L) \
    int bconv_##L(const BconvArgs* a, pc_stream_t s) { return bconv::launch<L>(a, s); }
PCH_BCONV_INST(12)
PCH_BCONV_INST(13)
PCH_BCONV_INST(14)
PCH_BCONV_INST(15)
PCH_BCONV_INST(16)
}  // namespace pch
