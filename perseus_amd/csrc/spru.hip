// The SPRU floating-point stages of the kernel table (crates/pc-kernels/kernels/spru.cuh, args.cuh:726-746): one
// forward Stockham pass of a batch of size-N complex transforms with table twiddles, and the scatter of FFT outputs
// into integer coefficient rows. Double precision throughout. The reference fixes where its products contract into
// fused multiply-adds (crates/pc-host/src/spru.rs:1-4, encode.rs:85-101); these kernels make exactly those fmas
// explicit and switch contraction off everywhere else, so the results are bit-identical to the reference's.
#include "common.h"

namespace pch {
namespace spru {

constexpr int BX = 256;

struct D2 {
    double x, y;
};

// j < N/2 of transform blockIdx.y: butterfly of (v0, v1) = (in[j], in[j + N/2]) with twiddle tw[(j % ns) (N/2) / ns]
// into out[idx], out[idx + ns], idx = (j / ns) 2 ns + j % ns (crates/pc-host/src/encode.rs:87-101, spru variant)
template <int LOGN>
__global__ void __launch_bounds__(BX) fft_pass_k(SpruFftArgs A, int lns) {
#pragma clang fp contract(off)
    constexpr uint32_t HALF = 1u << (LOGN - 1);
    const uint32_t j = blockIdx.x * BX + threadIdx.x;
    if (j >= HALF) return;
    const size_t e = (size_t)blockIdx.y << LOGN;
    const D2* in = (const D2*)A.in + e;
    D2* out = (D2*)A.out + e;
    const uint32_t ns = 1u << lns, k = j & (ns - 1);
    const D2 v0 = in[j], v1 = in[j + HALF];
    const D2 w = ((const D2*)A.tw)[k << (LOGN - 1 - lns)];
    const double tx = __builtin_fma(v1.x, w.x, -(v1.y * w.y));
    const double ty = __builtin_fma(v1.y, w.x, v1.x * w.y);
    const uint32_t idx = ((j >> lns) << (lns + 1)) + k;
    out[idx] = D2{v0.x + tx, v0.y + ty};
    out[idx + ns] = D2{v0.x - tx, v0.y - ty};
}

// coefficient k of FFT output blockIdx.y: m = rint(Re(y_k zt_k) / N * scale), its residues into limbs l < nl
// (crates/pc-host/src/spru.rs:110-140)
template <int LOGN>
__global__ void __launch_bounds__(BX) scatter_k(SpruScatterArgs A) {
#pragma clang fp contract(off)
    constexpr uint32_t N = 1u << LOGN;
    const uint32_t k = blockIdx.x * BX + threadIdx.x;
    if (k >= N) return;
    const size_t e = blockIdx.y;
    const D2 y = ((const D2*)A.y)[(e << LOGN) + k];
    const D2 z = ((const D2*)A.zt)[k];
    const double re = __builtin_fma(y.x, z.x, -(y.y * z.y)) * (1.0 / (double)N);
    const int64_t m = (int64_t)__builtin_rint(re * A.scale);
    const uint64_t am = m < 0 ? 0ull - (uint64_t)m : (uint64_t)m;
    uint32_t* out = (uint32_t*)A.out + e * A.out_stride + k;
    for (int l = 0; l < A.nl; ++l) {
        const uint64_t p = A.pr[l].p;
        uint64_t r = am % p;
        if (m < 0 && r != 0) r = p - r;
        out[(size_t)l << LOGN] = (uint32_t)r;
    }
}

template <int LOGN>
int fft_pass(const SpruFftArgs* a, pc_stream_t s) {
    constexpr int HALF = 1 << (LOGN - 1);
    if (!a || !a->in || !a->out || !a->tw || a->in == a->out) return -1;
    if (a->ns <= 0 || a->ns > HALF || (a->ns & (a->ns - 1)) || a->batch <= 0 || a->batch > 65535) return -1;
    const int lns = __builtin_ctz((unsigned)a->ns);
    hipLaunchKernelGGL(fft_pass_k<LOGN>, dim3((HALF + BX - 1) / BX, a->batch), dim3(BX), 0, (hipStream_t)s, *a, lns);
    return launch_rc();
}

template <int LOGN>
int scatter(const SpruScatterArgs* a, pc_stream_t s) {
    constexpr int N = 1 << LOGN;
    if (!a || !a->y || !a->out || !a->zt || !a->pr) return -1;
    if (a->nl <= 0 || a->batch <= 0 || a->batch > 65535) return -1;
    hipLaunchKernelGGL(scatter_k<LOGN>, dim3((N + BX - 1) / BX, a->batch), dim3(BX), 0, (hipStream_t)s, *a);
    return launch_rc();
}

}  // namespace spru

#define PCH_SPRU_INST(L)                                                                                  \
    int spru_fft_pass_##L(const SpruFftArgs* a, pc_stream_t s) { return spru::fft_pass<L>(a, s); }       \
    int spru_scatter_##L(const SpruScatterArgs* a, pc_stream_t s) { return spru::scatter<L>(a, s); }
PCH_SPRU_INST(12)
PCH_SPRU_INST(13)
PCH_SPRU_INST(14)
PCH_SPRU_INST(15)
PCH_SPRU_INST(16)

}  // namespace pch
