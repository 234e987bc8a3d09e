// The fixed device scratch of the allocation-free entry points (scratch.hip).
#ifndef SLM_SCRATCH_H
#define SLM_SCRATCH_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>

// Bytes of the array every GPU the library runs on holds until the process ends.
#define SLM_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)

// The current device's address of the array (hipGetSymbolAddress once per device).
hipError_t slm_scratch_address(void** out);

#endif
