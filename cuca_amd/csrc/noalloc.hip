// noalloc.hip -- the device scratch of the allocation-free entry points.
//
// cuca_hip_paged_decode_noalloc keeps its split-pass partials in this
// file-scope array instead of a caller's workspace, so a caller that cannot
// allocate (code under HIP graph capture, a serving loop that forbids
// hipMalloc) passes only its inputs and outputs.  Each GPU the library runs
// on holds its own copy of the array, at its own address, from the first
// context on that device until the process ends.
//
// The kernels live in the library's gfx950 code object and take the scratch
// as an ordinary pointer argument.  This file only defines the array and
// resolves its per-device address: it is compiled by hipcc (host and gfx950
// device code) so the HIP runtime registers the variable.
#include <hip/hip_runtime.h>

#include <mutex>

#include "noalloc.h"

static __device__ __align__(256) unsigned char scratch[CUCA_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_ptr[kMaxDevices];

}  // namespace

extern "C" hipError_t cuca_noalloc_scratch(int device, void **ptr) {
    if (!ptr) return hipErrorInvalidValue;
    *ptr = nullptr;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[device]) {
        int cur = -1;
        hipError_t e = hipGetDevice(&cur);
        if (e != hipSuccess) return e;
        if (cur != device) return hipErrorInvalidDevice;  // the caller makes the device current
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p || (reinterpret_cast<uintptr_t>(p) & 255u) != 0) return hipErrorInvalidSymbol;
        g_ptr[device] = p;
    }
    *ptr = g_ptr[device];
    return hipSuccess;
}
