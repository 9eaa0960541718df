// hsdpa_static.hip — the device scratch of hsdpa_attention_static: a
// file-scope array of HSDPA_STATIC_SCRATCH_BYTES that every GPU the library
// runs on holds until the process ends, for callers that cannot allocate
// (code under HIP graph capture, serving loops, harnesses that forbid
// hipMalloc). Its device address comes from hipGetSymbolAddress, once per
// device with that device current; host code never uses the array's name as
// an address (in host code it is a stand-in, not device memory).

#include <hip/hip_runtime.h>

#include <mutex>

#include "hsdpa.h"
#include "hsdpa_kernels.h"

static __device__ __align__(256) unsigned char scratch[HSDPA_STATIC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];

}  // namespace

namespace hsdpa {

hipError_t static_scratch(void **ptr)
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return hipSuccess;
}

}  // namespace hsdpa
