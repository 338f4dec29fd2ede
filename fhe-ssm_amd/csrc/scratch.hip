// scratch.hip -- the device scratch behind the allocation-free entry point (ckks_eval_mult_rescale_noalloc).
//
// One file-scope device array of kScratchBytes per GPU, held by every GPU the library runs on until the process
// ends.  Host code never passes the array's name to a kernel (on the host it is only a stand-in for the symbol):
// scratch_init() resolves the array's device address once per device, with that device current, and every later
// use goes through that address (scratch_ptr).  Calls that use the scratch on one GPU share it: two such calls in
// flight at once on one GPU (different streams or host threads) race.
#include <mutex>
#include <string.h>

#include "engine.hpp"

namespace fhe {

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
uint8_t* g_ptr[kMaxDevices] = {};

// a run of words written into device memory from the kernel's own arguments (no host staging, no allocation)
constexpr uint32_t kPutWords = 448;
struct PutChunk {
    uint32_t n;
    uint64_t w[kPutWords];
};

__global__ __launch_bounds__(256) void k_put_words(uint64_t* __restrict__ dst, PutChunk c) {
    for (uint32_t i = threadIdx.x; i < c.n; i += blockDim.x) dst[i] = c.w[i];
}

}  // namespace

hipError_t scratch_init(int device) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_ptr[device]) return hipSuccess;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_ptr[device] = (uint8_t*)p;
    return hipSuccess;
}

uint8_t* scratch_ptr(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lk(g_mu);
    return g_ptr[device];
}

hipError_t arena_put(void* dst, const void* src, size_t bytes, hipStream_t st) {
    if (bytes % 8) return hipErrorInvalidValue;
    const uint64_t* s = (const uint64_t*)src;
    uint64_t* d = (uint64_t*)dst;
    for (size_t w = 0, n = bytes / 8; w < n; w += kPutWords) {
        PutChunk c;
        c.n = (uint32_t)std::min<size_t>(kPutWords, n - w);
        memcpy(c.w, s + w, (size_t)c.n * 8);
        hipLaunchKernelGGL(k_put_words, dim3(1), dim3(256), 0, st, d + w, c);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace fhe
