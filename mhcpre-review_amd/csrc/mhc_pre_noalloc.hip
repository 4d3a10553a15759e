// Built-in workspace for callers that cannot allocate device memory (code
// under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc): a fixed array in the library's device code object, used by
// mhcPreNoAlloc in place of a caller-owned workspace.
//
// Each device the library runs on holds its own copy of the array until the
// process ends, at its own address; host code never passes the array's name
// to a kernel (on the host that name is only a stand-in for the symbol, not a
// device address) but the address hipGetSymbolAddress returns for the current
// device, looked up once per device.  Every launch on a device shares that
// device's copy and finds the previous launch's contents there; the kernels
// need nothing in it to start at zero (the exchange tags carry an epoch kept
// in the array's header, the split-K partials are written before they are
// read).  Launches that overlap on one device race on the array.

#include "mhc_pre_internal.h"

#include <hip/hip_runtime.h>

#include <mutex>

namespace {

static __device__ __align__(256) unsigned char scratch[mhc::kScratchBytes];

}  // namespace

namespace mhc {

hipError_t scratch_address(int device, void **ptr)
{
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static void *addr[kMaxDevices] = {};
    if (device < 0 || device >= kMaxDevices || ptr == nullptr) {
        return hipErrorInvalidValue;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (addr[device] == nullptr) {
        // The caller has made `device` current: the symbol resolves to that
        // device's copy of the array.
        void *p = nullptr;
        const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess) {
            return err;
        }
        if (p == nullptr) {
            return hipErrorInvalidSymbol;
        }
        addr[device] = p;
    }
    *ptr = addr[device];
    return hipSuccess;
}

}  // namespace mhc
