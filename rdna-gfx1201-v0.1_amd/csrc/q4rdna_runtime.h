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

// How a per-tensor GEMV launches: the VALU kernel's split-K factor and the
// exchange slots (words, zero between launches) its K chunks meet in; none
// when the K dimension is not split.
struct TensorLaunch {
    uint32_t split;
    size_t slots;
    bool sequential;  // Q4RDNA_KERNEL_SEQUENTIAL: split 1, no workspace
};

// Validate q4rdna_mul_mat_ex's arguments (the same statuses as that entry
// point) and resolve how it launches.
int check_mul_mat_ex(const q4rdna_weight *w, const q4rdna_weight *gate, const float *x, const float *add,
                     const float *y, const q4rdna_launch_options *options, TensorLaunch *launch);

// Launch a validated per-tensor GEMV with caller-provided exchange slots: at
// least launch.slots words (ignored when that is zero), zero on entry and
// left zero.
// Count one GEMV launch over W (and its SwiGLU gate, may be null) in the
// library's launch statistics (q4rdna_launch_count, q4rdna_sidecar_hits).
// Allocates nothing.
void count_gemv_launch(const uint8_t *w, const uint8_t *gate);

int launch_tensor_in(const TensorLaunch &launch, const q4rdna_weight *w, const uint8_t *gate, const float *x,
                     const float *add, float *y, uint32_t *slots, hipStream_t stream);

}  // namespace q4rdna
