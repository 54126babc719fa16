// Opt-in kernel timing used by benchmarks: while a family is enabled, its launches are
// bracketed by HIP events recorded on the launch stream (see ct_profile_begin).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ct {

// Returns a slot index, or -1 when the family is not being timed (the common case: one
// relaxed atomic load).
int profile_open(int family, hipStream_t stream);
// Records the stop event of slot `slot` and the launch's algorithmic work.
void profile_close(int slot, hipStream_t stream, double work);

}  // namespace ct
