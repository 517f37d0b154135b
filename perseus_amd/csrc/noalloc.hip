// The rotate-and-sum ladder for callers that cannot allocate device memory (code under HIP graph capture, tight
// serving loops, harnesses that forbid allocation): pcx_rotate_and_sum with its scratch ciphertext in a file-scope
// device array instead of a caller's buffer. The array holds PCX_NOALLOC_SCRATCH_WORDS u32 words (32 MiB: a
// ciphertext of 2 parts x 64 rows x 2^16 words) on every device the library runs on, until the process ends.
//
// Host code never passes the array's name to a kernel: each device's address comes from hipGetSymbolAddress, taken
// once per device with that device current (at context creation, pcx_ctx_new_k), and only that address reaches the
// launches.
#include <hip/hip_runtime.h>

#include <mutex>

#include "pc_hip.h"

namespace {

__device__ __align__(256) uint32_t scratch[PCX_NOALLOC_SCRATCH_WORDS];

constexpr int MAX_DEV = 64;
std::mutex g_mu;
void* g_ptr[MAX_DEV];

// the current device's address of `scratch` (looked up once per device), or null with *rc set
void* scratch_ptr(int* rc) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEV) {
        *rc = -1;
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            *rc = e != hipSuccess ? (int)e : -1;
            return nullptr;
        }
        g_ptr[dev] = p;
    }
    return g_ptr[dev];
}

}  // namespace

namespace pch {
// Called by pcx_ctx_new_k with the context's device current: the address is looked up at set-up, outside any stream
// capture a caller may later run the entry point under (a first lookup can load the code object, which a capture may
// refuse). Returns 0 or the lookup's error; the entry point retries a failed lookup on its first call.
int noalloc_prepare() {
    int rc = 0;
    return scratch_ptr(&rc) ? 0 : rc;
}
}  // namespace pch

extern "C" int pcx_rotate_and_sum_noalloc(pcx_ctx* c, pcx_keys* k, const void* x, int top, int64_t start,
                                          int64_t stop, int radix_bits, void* out, pc_stream_t s) {
    if (!c) return -1;
    if (pcx_ct_words(c) > (size_t)PCX_NOALLOC_SCRATCH_WORDS || radix_bits > 8) return -2;
    int rc = 0;
    void* tmp = scratch_ptr(&rc);
    if (!tmp) return rc;
    // every rotation the ladder writes into the scratch covers the rows it then reads (rows 0..top of both parts), so
    // what a previous call left there is never read
    return pcx_rotate_and_sum(c, k, x, top, start, stop, radix_bits, out, tmp, s);
}
