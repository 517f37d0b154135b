// Element-wise kernels over polynomial row sets and the eval-form automorphism (crates/pc-kernels/kernels/args.cuh
// EwArgs :143-160, AutomorphArgs :582-592; host twin crates/pc-host/src/elem.rs). Grid (N / 1024, rows of the row set,
// K x nparts), 256 threads of 4 consecutive words (16-byte accesses; rows are N-word aligned).
#include "common.h"

namespace pch {
namespace elem {

constexpr int BX = 256;

__device__ __forceinline__ int rs_row(const RowSet& rs, int y) { return y < rs.nq ? y : rs.qmax + (y - rs.nq); }
__device__ __forceinline__ uint32_t* at(const PolyRef& r, int c, int part, int row, int logn) {
    return (uint32_t*)r.base + c * r.ct_stride + part * r.part_stride + ((size_t)row << logn);
}

// op 0 add / sub, 1 scale, 2 sub_mul, 3 copy
template <int OP>
__global__ void __launch_bounds__(BX) ew_k(EwArgs A, int logn) {
    const int y = blockIdx.y;
    const int row = rs_row(A.rs, y);
    const int c = blockIdx.z / A.nparts, part = blockIdx.z % A.nparts;
    const uint32_t i = (blockIdx.x * BX + threadIdx.x) * 4;
    uint32_t* o = at(A.out, c, part, row, logn) + i;
    if (OP == 3) {
        *(uint4*)o = *(const uint4*)(at(A.a, c, part, row, logn) + i);
        return;
    }
    const uint32_t p = (uint32_t)A.pr[row].p;
    if (OP == 1 && A.zero_p && y >= A.rs.nq) {
        *(uint4*)o = make_uint4(0, 0, 0, 0);
        return;
    }
    const uint4 x4 = *(const uint4*)(at(A.a, c, part, row, logn) + i);
    uint32_t x[4] = {x4.x, x4.y, x4.z, x4.w}, r[4];
    if (OP == 0 || OP == 2) {
        const uint4 y4 = *(const uint4*)(at(A.b, c, part, row, logn) + i);
        const uint32_t yv[4] = {y4.x, y4.y, y4.z, y4.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) r[k] = (OP == 0 && !A.sub) ? addm(x[k], yv[k], p) : subm(x[k], yv[k], p);
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) r[k] = x[k];
    }
    if (OP == 1 || OP == 2) {
        const uint32_t s = ((const uint32_t*)A.sc)[row], ss = ((const uint32_t*)A.scs)[row];
#pragma unroll
        for (int k = 0; k < 4; ++k) r[k] = shoup(r[k], s, ss, p);
    }
    *(uint4*)o = make_uint4(r[0], r[1], r[2], r[3]);
}

template <int OP, int LOGN>
int ew(const EwArgs* a, pc_stream_t s) {
    if (!a || !a->out.base || !a->a.base || a->K < 0 || a->nparts < 0) return -1;
    if ((OP == 0 || OP == 2) && !a->b.base) return -1;
    if ((OP == 1 || OP == 2) && (!a->sc || !a->scs)) return -1;
    if (OP != 3 && !a->pr) return -1;
    const int rows = a->rs.nq + a->rs.np;
    if (rows <= 0 || a->K == 0 || a->nparts == 0) return 0;
    hipLaunchKernelGGL(ew_k<OP>, dim3((1 << LOGN) / (BX * 4), rows, a->K * a->nparts), dim3(BX), 0, (hipStream_t)s, *a,
                       LOGN);
    return launch_rc();
}

// out[o] = in[automorph_slot(k, o)] (+ add[o]); a gather: every 32-slot aligned block of the output reads one
// 32-slot aligned block of the input
template <bool ADD>
__global__ void __launch_bounds__(BX) automorph_k(AutomorphArgs A, int logn) {
    const int row = rs_row(A.rs, blockIdx.y);
    const int c = blockIdx.z / A.nparts, part = blockIdx.z % A.nparts;
    const uint32_t o = blockIdx.x * BX + threadIdx.x;
    uint32_t v = at(A.in, c, part, row, logn)[automorph_slot(A.k, o, logn)];
    if (ADD) v = addm(v, at(A.add, c, part, row, logn)[o], (uint32_t)A.pr[row].p);
    at(A.out, c, part, row, logn)[o] = v;
}

template <int LOGN>
int automorph(const AutomorphArgs* a, pc_stream_t s) {
    if (!a || (a->k & 1u) == 0 || !a->out.base || !a->in.base) return -1;
    if (a->has_add && (!a->add.base || !a->pr)) return -1;
    const int rows = a->rs.nq + a->rs.np;
    if (rows <= 0 || a->K <= 0 || a->nparts <= 0) return 0;
    const dim3 grid((1 << LOGN) / BX, rows, a->K * a->nparts);
    if (a->has_add) hipLaunchKernelGGL(automorph_k<true>, grid, dim3(BX), 0, (hipStream_t)s, *a, LOGN);
    else hipLaunchKernelGGL(automorph_k<false>, grid, dim3(BX), 0, (hipStream_t)s, *a, LOGN);
    return launch_rc();
}

}  // namespace elem

#define PCH_EW_INST(L)                                                                                \
    int ew_add_##L(const EwArgs* a, pc_stream_t s) { return elem::ew<0, L>(a, s); }                  \
    int ew_scale_##L(const EwArgs* a, pc_stream_t s) { return elem::ew<1, L>(a, s); }                \
    int ew_sub_mul_##L(const EwArgs* a, pc_stream_t s) { return elem::ew<2, L>(a, s); }              \
    int ew_copy_##L(const EwArgs* a, pc_stream_t s) { return elem::ew<3, L>(a, s); }                 \
    int automorph_##L(const AutomorphArgs* a, pc_stream_t s) { return elem::automorph<L>(a, s); }
PCH_EW_INST(12)
PCH_EW_INST(13)
PCH_EW_INST(14)
PCH_EW_INST(15)
PCH_EW_INST(16)

}  // namespace pch

// ------------------------------------------------------------------------------------------------ HBM copy probe
// A plain stream copy of a known byte count: each 256-thread block moves one contiguous 16 KiB tile, every thread four
// 16-byte words at stride 4 KiB. It measures the achievable HBM bandwidth and calibrates the FETCH_SIZE / WRITE_SIZE
// counters (their reading for this kernel over the bytes it must move).
namespace pch {
namespace elem {
__global__ void __launch_bounds__(BX) copy_probe_k(uint4* __restrict__ dst, const uint4* __restrict__ src) {
    const size_t base = (size_t)blockIdx.x * (BX * 4) + threadIdx.x;
    uint4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = src[base + k * BX];
#pragma unroll
    for (int k = 0; k < 4; ++k) dst[base + k * BX] = v[k];
}
}  // namespace elem
}  // namespace pch

extern "C" int pcx_copy_probe(void* dst, const void* src, size_t bytes, pc_stream_t s) {
    constexpr size_t TILE = pch::elem::BX * 4 * 16;
    if (!dst || !src || bytes == 0 || bytes % TILE || bytes / TILE > 0x7fffffffu) return -1;
    hipLaunchKernelGGL(pch::elem::copy_probe_k, dim3((unsigned)(bytes / TILE)), dim3(pch::elem::BX), 0,
                       (hipStream_t)s, (uint4*)dst, (const uint4*)src);
    return pch::launch_rc();
}

// ------------------------------------------------------------------------------------------------ VALU probe
// The throughput of single VALU instruction forms: each thread runs `iters` rounds of 8 independent dependency chains
// of one form (inline assembly, so that the instruction is the one named), a workgroup of 256 threads; the wave-
// instructions issued are 8 iters per wave. Timed by the caller, it states what the integer work of the kernels can
// reach beside the spec figures: the kernels' products (v_mul_lo/hi_u32, v_mad_u64_u32), ChaCha12's add / xor / rotate
// (v_alignbit_b32) and the conditional subtraction's v_min_u32. Nothing is read; one word per thread is written only
// when the chains end on a value they never reach (so the work is not removed), inside the caller's 1024 words.
namespace pch {
namespace elem {
template <int K>
__global__ void __launch_bounds__(BX) valu_probe_k(uint32_t* out, int iters, uint32_t seed) {
    uint32_t x[8];
    uint64_t y[8];
    const uint32_t t = blockIdx.x * BX + threadIdx.x;
    const uint32_t c = seed | 1u;
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = (t + seed) * (2u * i + 3u) | 1u, y[i] = x[i];
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if constexpr (K == 0) asm volatile("v_add_u32 %0, %0, %1" : "+v"(x[i]) : "v"(c));
            if constexpr (K == 1) asm volatile("v_xor_b32 %0, %0, %1" : "+v"(x[i]) : "v"(c));
            if constexpr (K == 2) asm volatile("v_alignbit_b32 %0, %0, %0, 16" : "+v"(x[i]));
            if constexpr (K == 3) asm volatile("v_min_u32 %0, %0, %1" : "+v"(x[i]) : "v"(c));
            if constexpr (K == 4) asm volatile("v_mul_lo_u32 %0, %0, %1" : "+v"(x[i]) : "v"(c));
            if constexpr (K == 5) asm volatile("v_mul_hi_u32 %0, %0, %1" : "+v"(x[i]) : "v"(c));
            if constexpr (K == 6) {
                uint64_t cc;
                asm volatile("v_mad_u64_u32 %0, %1, %2, %3, %0" : "+v"(y[i]), "=s"(cc) : "v"(x[i]), "v"(c));
            }
        }
    }
    uint32_t r = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) r ^= x[i] ^ (uint32_t)y[i] ^ (uint32_t)(y[i] >> 32);
    if (r == 0x9E3779B9u) out[t & 1023] = r;
}
}  // namespace elem
}  // namespace pch

extern "C" int pcx_valu_probe(int kind, int blocks, int iters, uint32_t* out, pc_stream_t s) {
    if (!out || blocks < 1 || iters < 1) return -1;
    hipStream_t st = (hipStream_t)s;
    const dim3 g((unsigned)blocks), b(pch::elem::BX);
    switch (kind) {
        case 0: hipLaunchKernelGGL(pch::elem::valu_probe_k<0>, g, b, 0, st, out, iters, 1u); break;
        case 1: hipLaunchKernelGGL(pch::elem::valu_probe_k<1>, g, b, 0, st, out, iters, 1u); break;
        case 2: hipLaunchKernelGGL(pch::elem::valu_probe_k<2>, g, b, 0, st, out, iters, 1u); break;
        case 3: hipLaunchKernelGGL(pch::elem::valu_probe_k<3>, g, b, 0, st, out, iters, 1u); break;
        case 4: hipLaunchKernelGGL(pch::elem::valu_probe_k<4>, g, b, 0, st, out, iters, 1u); break;
        case 5: hipLaunchKernelGGL(pch::elem::valu_probe_k<5>, g, b, 0, st, out, iters, 1u); break;
        case 6: hipLaunchKernelGGL(pch::elem::valu_probe_k<6>, g, b, 0, st, out, iters, 1u); break;
        default: return -1;
    }
    return pch::launch_rc();
}

// ------------------------------------------------------------------------------------------------ byte fill
// cudaMemsetAsync's replacement (crates/pc-cuda/src/mem.rs:305-331, DBuf::zero / zero_range) as an ordinary kernel, so
// that a replay captured into a HIP graph holds a kernel node and no memset node. The body between the first and
// last 16-byte boundaries is written with 16-byte stores (grid-stride); the head and tail bytes (< 16 each) by one
// thread.
namespace pch {
namespace elem {
__global__ void __launch_bounds__(BX) fill_k(uint8_t* dst, uint32_t pat, size_t head, size_t body16, size_t tail) {
    const size_t tid = (size_t)blockIdx.x * BX + threadIdx.x, stride = (size_t)gridDim.x * BX;
    uint4* b = (uint4*)(dst + head);
    const uint4 v = make_uint4(pat, pat, pat, pat);
    for (size_t i = tid; i < body16; i += stride) b[i] = v;
    if (tid == 0) {
        const uint8_t c = (uint8_t)pat;
        for (size_t i = 0; i < head; ++i) dst[i] = c;
        uint8_t* t = dst + head + body16 * 16;
        for (size_t i = 0; i < tail; ++i) t[i] = c;
    }
}
}  // namespace elem

int fill_bytes(void* dst, int value, size_t bytes, pc_stream_t s) {
    if (bytes == 0) return 0;
    if (!dst) return -1;
    uint8_t* d = (uint8_t*)dst;
    size_t head = (16 - ((uintptr_t)d & 15)) & 15;
    if (head > bytes) head = bytes;
    const size_t body16 = (bytes - head) / 16, tail = bytes - head - body16 * 16;
    const uint32_t c = (uint32_t)(value & 0xFF);
    const size_t want = (body16 + elem::BX - 1) / elem::BX;
    const unsigned grid = (unsigned)(want < 1 ? 1 : want > 4096 ? 4096 : want);
    hipLaunchKernelGGL(elem::fill_k, dim3(grid), dim3(elem::BX), 0, (hipStream_t)s, d, c * 0x01010101u, head, body16,
                       tail);
    return launch_rc();
}
}  // namespace pch
