// Runtime helpers shared by the host runtime (q4rdna_runtime.cpp) and the
// allocation-free entry point (q4rdna_noalloc.hip).  Not part of the C ABI.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#include "q4rdna.h"

namespace q4rdna {

// Record `fmt` as the calling thread's last error; returns `code`.
int set_error(int code, const char *fmt, ...);

// Validate q4rdna_mul_mat_ex's arguments (the same statuses as that entry
// point) and resolve the split-K factor it launches with.
int check_mul_mat_ex(const q4rdna_weight *w, const q4rdna_weight *gate, const float *x, const float *add,
                     const float *y, const q4rdna_launch_options *options, uint32_t *split);

// Workspace a per-tensor launch with that split needs: fp32 partials and
// arrival counters (none when split == 1).
void gemv_workspace_need(const q4rdna_weight *w, bool gate, uint32_t split, size_t *partial_floats,
                         size_t *counters);

// Launch a validated per-tensor GEMV with a caller-provided workspace of at
// least gemv_workspace_need() (ignored when split == 1); counters zero on
// entry, left zero.
int launch_gemv_in(const q4rdna_weight *w, const uint8_t *gate, const float *x, const float *add, float *y,
                   uint32_t split, float *partial, uint32_t *counters, hipStream_t stream);

}  // namespace q4rdna
