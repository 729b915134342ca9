// The scratch of og_int8_gemm_noalloc: one fixed array per device, so that the entry point allocates nothing (for
// callers under HIP graph capture or in loops that may not call hipMalloc). Its device address is looked up once per
// device, with that device current (og_init), and kept; host code uses that address, never the array's name (which on
// the host is only a stand-in for the symbol).
//
// Layout: the first kNoAllocWordBytes hold the one-launch few-rows kernel's count words, which must be zero before a
// launch; they are cleared here once, at set-up, and every launch leaves them zero. The rest holds partial sums,
// which every product writes before it reads them. Every call on a device shares the array: calls that overlap on one
// device race.
#include <mutex>

#include "og_internal.hpp"

namespace og {

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mutex;
void *g_scratch[kMaxDevices];

}  // namespace

hipError_t noalloc_scratch_setup(int device, hipStream_t s, void **out)
{
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!g_scratch[device]) {
        void *p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        e = launch_fill_bytes(p, 0, kNoAllocWordBytes, s);   // the count words start at zero
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) return e;
        g_scratch[device] = p;
    }
    *out = g_scratch[device];
    return hipSuccess;
}

}  // namespace og
