// CKKS slot encoding on the device (the table's `encode` entry; semantics crates/pc-kernels/kernels/args.cuh EncodeArgs
// and encode.cuh, driven by crates/pc-gpu/src/encode_dev.rs fft_v): N/2 complex slots v_j -> N coefficient-form rows.
//   1. slot j sits at the odd power t = 5^j mod 2N of zeta = exp(i pi / N), its conjugate at 2N - t: w[(t - 1) / 2] = v_j,
//      w[(2N - t - 1) / 2] = conj(v_j);
//   2. Y = DFT_N(w) (exp(-2 pi i n k / N)), here as a four-step transform N = N1 N2 in two LDS kernels (N1-point
//      transforms down the columns, the twiddle W_N^(n2 k1), N2-point transforms along the rows);
//   3. c_k = scale Re(Y_k zeta^-k) / N, and max |c_k| (non-negative doubles order as their bit patterns);
//   4. split = ceil(log2 max |c|) - 61 when positive (OpenFHE's 2^61 split), m_k = round(c_k / 2^split) half away from
//      zero, out[l][k] = (m_k mod p_l) * deg_factor[l] * 2^split mod p_l.
// Twiddles are sin / cos of pi a / 2^b for integers a, b, computed here (sincospi_dyadic): the angle is reduced exactly
// (integer arithmetic on a) to [0, pi/4], then Taylor series of sin and cos evaluated by Horner's rule in double.
// Floating-point words may differ from the reference's (its twiddles come from another sin/cos and another FFT order);
// the rounded coefficients agree with any exact encoder except where the transform's double error (~1e-5 coefficient
// units at scale 2^40, N = 2^16) straddles a half, the tolerance the reference states between its host and device
// encoders (encode_dev.rs:1-9).
#include "common.h"

namespace pch {
namespace enc {

constexpr int BX = 256;
constexpr int CPW = 4;  // columns (rows) per workgroup of the two transform kernels

constexpr double fact(int n) { return n <= 1 ? 1.0 : n * fact(n - 1); }  // exact in double up to 22!

// sin(pi a / 2^b), cos(pi a / 2^b)
__device__ __forceinline__ void sincospi_dyadic(long long a, int b, double& s, double& c) {
    // lift to b >= 2 so that a quadrant and an octant are whole numbers of units
    if (b < 2) {
        a <<= (2 - b);
        b = 2;
    }
    const long long full = 1LL << (b + 1), quad = 1LL << (b - 1), oct = 1LL << (b - 2);
    long long u = a & (full - 1);  // [0, 2 pi)
    const int q = (int)(u / quad);
    long long r = u - (long long)q * quad;  // [0, pi/2)
    const bool swap = r > oct;
    if (swap) r = quad - r;  // [0, pi/4]
    // phi = pi r / 2^b, with pi as a double pair (the angle to about 2^-105 relative)
    const double x = (double)r * ldexp(1.0, -b);
    const double pi_hi = 3.141592653589793116, pi_lo = 1.2246467991473532e-16;
    const double t = x * pi_hi;
    const double phi = t + (__fma_rn(x, pi_hi, -t) + x * pi_lo);
    const double z = phi * phi;
    // Taylor series to phi^19 / 19! and phi^20 / 20!: the first omitted terms are below 1e-22 at phi <= pi / 4
    double ps = -1.0 / fact(19);
    ps = __fma_rn(ps, z, 1.0 / fact(17));
    ps = __fma_rn(ps, z, -1.0 / fact(15));
    ps = __fma_rn(ps, z, 1.0 / fact(13));
    ps = __fma_rn(ps, z, -1.0 / fact(11));
    ps = __fma_rn(ps, z, 1.0 / fact(9));
    ps = __fma_rn(ps, z, -1.0 / fact(7));
    ps = __fma_rn(ps, z, 1.0 / fact(5));
    ps = __fma_rn(ps, z, -1.0 / fact(3));
    const double sn = __fma_rn(ps * z, phi, phi);
    double pc = 1.0 / fact(20);
    pc = __fma_rn(pc, z, -1.0 / fact(18));
    pc = __fma_rn(pc, z, 1.0 / fact(16));
    pc = __fma_rn(pc, z, -1.0 / fact(14));
    pc = __fma_rn(pc, z, 1.0 / fact(12));
    pc = __fma_rn(pc, z, -1.0 / fact(10));
    pc = __fma_rn(pc, z, 1.0 / fact(8));
    pc = __fma_rn(pc, z, -1.0 / fact(6));
    pc = __fma_rn(pc, z, 1.0 / fact(4));
    pc = __fma_rn(pc, z, -1.0 / fact(2));
    const double cs = __fma_rn(pc, z, 1.0);
    double s0 = swap ? cs : sn, c0 = swap ? sn : cs;
    switch (q) {
        case 0: s = s0, c = c0; break;
        case 1: s = c0, c = -s0; break;
        case 2: s = -s0, c = -c0; break;
        default: s = -c0, c = s0; break;
    }
}

// exp(-2 pi i e / 2^lg) for 0 <= e < 2^lg
__device__ __forceinline__ double2 root(long long e, int lg) {
    double s, c;
    sincospi_dyadic(-2 * e, lg, s, c);
    return make_double2(c, s);
}
__device__ __forceinline__ double2 cmul(double2 a, double2 b) {
    return make_double2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}

// 1. slot placement (one thread per slot)
__global__ void __launch_bounds__(BX) place_k(const double2* v, double2* w, int logn) {
    const uint32_t n = 1u << logn, j = blockIdx.x * BX + threadIdx.x;
    if (j >= n / 2) return;
    const uint32_t m2n = 2 * n - 1;
    uint32_t t = 1, b = 5, e = j;
    while (e) {
        if (e & 1u) t = (t * b) & m2n;
        b = (b * b) & m2n;
        e >>= 1;
    }
    const double2 x = v[j];
    w[(t - 1) / 2] = x;
    w[(2 * n - t - 1) / 2] = make_double2(x.x, -x.y);
}

// In-LDS transforms of CPW sequences of L = 2^lg points (sequence q at s[q L ...]): natural order in and out,
// bit-reversal then radix-2 Cooley-Tukey stages.
__device__ void dft_lds(double2* s, int lg) {
    const int L = 1 << lg, tot = CPW * L;
    for (int e = threadIdx.x; e < tot; e += BX) {
        const int q = e >> lg, i = e & (L - 1), j = (int)(__brev((uint32_t)i) >> (32 - lg));
        if (i < j) {
            const double2 a = s[q * L + i];
            s[q * L + i] = s[q * L + j];
            s[q * L + j] = a;
        }
    }
    __syncthreads();
    for (int lh = 0; lh < lg; ++lh) {
        const int h = 1 << lh;
        for (int e = threadIdx.x; e < tot / 2; e += BX) {
            const int q = e >> (lg - 1), bb = e & (L / 2 - 1), r = bb & (h - 1);
            const int i0 = q * L + ((bb >> lh) << (lh + 1)) + r, i1 = i0 + h;
            const double2 t = cmul(s[i1], root(r, lh + 1));
            const double2 u = s[i0];
            s[i0] = make_double2(u.x + t.x, u.y + t.y);
            s[i1] = make_double2(u.x - t.x, u.y - t.y);
        }
        __syncthreads();
    }
}

// 2a. columns: x[n1 N2 + n2] for the workgroup's CPW columns n2, N1-point transforms, times W_N^(n2 k1); written as
//     X[k1 N2 + n2]
__global__ void __launch_bounds__(BX) cols_k(const double2* x, double2* X, int lg1, int lg2) {
    extern __shared__ double2 s[];
    const int N1 = 1 << lg1, N2 = 1 << lg2, c0 = blockIdx.x * CPW;
    for (int e = threadIdx.x; e < CPW * N1; e += BX) {
        const int n1 = e / CPW, q = e % CPW;
        s[q * N1 + n1] = x[(size_t)n1 * N2 + c0 + q];
    }
    __syncthreads();
    dft_lds(s, lg1);
    for (int e = threadIdx.x; e < CPW * N1; e += BX) {
        const int k1 = e / CPW, q = e % CPW, n2 = c0 + q;
        const long long ex = ((long long)n2 * k1) & ((1LL << (lg1 + lg2)) - 1);
        X[(size_t)k1 * N2 + n2] = cmul(s[q * N1 + k1], root(ex, lg1 + lg2));
    }
}

// 2b. rows: X[k1 N2 + n2] for the workgroup's CPW rows k1, N2-point transforms; Y[k1 + N1 k2]
__global__ void __launch_bounds__(BX) rows_k(const double2* X, double2* Y, int lg1, int lg2) {
    extern __shared__ double2 s[];
    const int N1 = 1 << lg1, N2 = 1 << lg2, r0 = blockIdx.x * CPW;
    for (int e = threadIdx.x; e < CPW * N2; e += BX) {
        const int q = e / N2, n2 = e % N2;
        s[q * N2 + n2] = X[(size_t)(r0 + q) * N2 + n2];
    }
    __syncthreads();
    dft_lds(s, lg2);
    for (int e = threadIdx.x; e < CPW * N2; e += BX) {
        const int k2 = e / CPW, q = e % CPW;
        Y[(size_t)(r0 + q) + (size_t)N1 * k2] = s[q * N2 + k2];
    }
}

// 3. coefficients and their largest magnitude (cmax cleared by clear_k first, on the same stream)
__global__ void clear_k(unsigned long long* cmax) { *cmax = 0; }
__global__ void __launch_bounds__(BX) coef_k(const double2* Y, double scale, double* c, unsigned long long* cmax,
                                             int logn) {
    const int n = 1 << logn, k = blockIdx.x * BX + threadIdx.x;
    double a = 0.0;
    if (k < n) {
        double sn, cs;
        sincospi_dyadic(-(long long)k, logn, sn, cs);
        const double re = (Y[k].x * cs - Y[k].y * sn) / (double)n * scale;
        c[k] = re;
        a = fabs(re);
    }
    // wave maximum, then one atomic per wave
    for (int o = 32; o > 0; o >>= 1) a = fmax(a, __shfl_xor(a, o));
    if ((threadIdx.x & 63) == 0) atomicMax(cmax, (unsigned long long)__double_as_longlong(a));
}

// 4. residues: OpenFHE's split, rounding half away from zero, one modular product per prime
__global__ void __launch_bounds__(BX) scatter_k(const double* c, const unsigned long long* cmax, uint32_t* out,
                                                const uint32_t* deg_factor, const PrimeConst* pr, int nl, int logn) {
    const int n = 1 << logn, k = blockIdx.x * BX + threadIdx.x;
    if (k >= n) return;
    const double mx = __longlong_as_double((long long)*cmax);
    int split = 0;
    if (mx > 0.0) {
        int e;
        const double f = frexp(mx, &e);  // mx = f 2^e, f in [1/2, 1): ceil(log2 mx) = e, or e - 1 at f = 1/2
        const int logc = f == 0.5 ? e - 1 : e;
        split = logc > 61 ? logc - 61 : 0;
    }
    const long long m = llround(ldexp(c[k], -split));
    const uint64_t am = m < 0 ? (uint64_t)(-(m + 1)) + 1 : (uint64_t)m;
    for (int l = 0; l < nl; ++l) {
        const Red red(pr[l]);
        uint32_t f = deg_factor[l];
        for (int i = 0; i < split; ++i) f = addm(f, f, red.p);
        uint32_t r = red(am);
        if (m < 0 && r) r = red.p - r;
        out[((size_t)l << logn) + k] = red.mul(r, f);
    }
}

}  // namespace enc

template <int LOGN>
int encode(const EncodeArgs* a, pc_stream_t s) {
    if (!a || !a->v || !a->a || !a->b || !a->c || !a->cmax || !a->out || !a->deg_factor || !a->pr || a->nl < 0)
        return -1;
    if (!(a->scale > 0.0)) return -1;
    if (a->nl == 0) return 0;
    constexpr int N = 1 << LOGN, LG1 = (LOGN + 1) / 2, LG2 = LOGN - LG1;
    hipStream_t st = (hipStream_t)s;
    double2* A = (double2*)a->a;
    double2* B = (double2*)a->b;
    hipLaunchKernelGGL(enc::place_k, dim3((N / 2 + enc::BX - 1) / enc::BX), dim3(enc::BX), 0, st, (const double2*)a->v,
                       A, LOGN);
    hipLaunchKernelGGL(enc::cols_k, dim3((1 << LG2) / enc::CPW), dim3(enc::BX),
                       enc::CPW * (1 << LG1) * sizeof(double2), st, (const double2*)A, B, LG1, LG2);
    hipLaunchKernelGGL(enc::rows_k, dim3((1 << LG1) / enc::CPW), dim3(enc::BX),
                       enc::CPW * (1 << LG2) * sizeof(double2), st, (const double2*)B, A, LG1, LG2);
    hipLaunchKernelGGL(enc::clear_k, dim3(1), dim3(1), 0, st, a->cmax);
    hipLaunchKernelGGL(enc::coef_k, dim3((N + enc::BX - 1) / enc::BX), dim3(enc::BX), 0, st, (const double2*)A,
                       a->scale, (double*)a->c, a->cmax, LOGN);
    hipLaunchKernelGGL(enc::scatter_k, dim3((N + enc::BX - 1) / enc::BX), dim3(enc::BX), 0, st, (const double*)a->c,
                       (const unsigned long long*)a->cmax, (uint32_t*)a->out, (const uint32_t*)a->deg_factor, a->pr,
                       a->nl, LOGN);
    return launch_rc();
}

#define PCH_ENC_INST(L) \
    int encode_##L(const EncodeArgs* a, pc_stream_t s) { return encode<L>(a, s); }
PCH_ENC_INST(12)
PCH_ENC_INST(13)
PCH_ENC_INST(14)
PCH_ENC_INST(15)
PCH_ENC_INST(16)

}  // namespace pch
