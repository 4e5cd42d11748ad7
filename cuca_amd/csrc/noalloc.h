// noalloc.h -- the device scratch behind the allocation-free entry points
// (cuca_hip_paged_decode_noalloc), defined in noalloc.hip.
#ifndef CUCA_NOALLOC_H
#define CUCA_NOALLOC_H

#include <hip/hip_runtime_api.h>

#include "cuca_hip.h"  // CUCA_NOALLOC_SCRATCH_BYTES

#ifdef __cplusplus
extern "C" {
#endif

// The device address of this device's copy of the scratch array.  Call with
// `device` current; the address is resolved with hipGetSymbolAddress once per
// device and kept.  The array's own name is a host-side stand-in: kernels and
// copies take only the address returned here.
hipError_t cuca_noalloc_scratch(int device, void **ptr);

#ifdef __cplusplus
}
#endif
#endif
