// Per-device static scratch of the allocation-free decode step.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/libkrillhip.h"

namespace krill {

// Size of the static scratch: the split-K workspace of one decode step
// (8.7 MB for 40 query / 8 KV heads, D = 128, 32 sequences on a 256-CU
// device; that shape exceeds 32 MiB from 1,230 sequences on).
constexpr size_t kScratchBytes = KRILL_NOALLOC_SCRATCH_BYTES;
constexpr int kScratchMaxDevices = 64;

// Resolves `device`'s copy of the scratch array (hipGetSymbolAddress with
// `device` current, once per device; later calls return at once).
hipError_t scratch_init(int device);
// The device address resolved by scratch_init, or null before it.
void *scratch_ptr(int device);

}  // namespace krill
