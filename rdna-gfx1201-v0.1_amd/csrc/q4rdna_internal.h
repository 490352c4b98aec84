// Internal interface between the host runtime (q4rdna_runtime.cpp) and the
// gfx950 kernels (q4rdna_kernels.hip).  Not part of the C ABI.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

namespace q4rdna {

constexpr uint32_t kGroup = 64;
constexpr uint32_t kTileRows = 32;
constexpr uint32_t kTileBytes = 1088;

// One GEMV launch.  gate != nullptr selects SwiGLU, add != nullptr the bias
// epilogue.  split > 1 reduces K chunks across workgroups through
// partial[split * rows (x2 with gate)] and counters[rows / 32], which must be
// zero on entry and are left zero.
struct GemvArgs {
    const uint8_t *w;
    const uint8_t *gate;
    const float *x;
    const float *add;
    float *y;
    uint32_t rows;
    uint32_t cols;
    uint32_t split;
    float *partial;
    uint32_t *counters;
};

// Device-side descriptor of one GEMV in a multi-tensor plan.
struct PlanDesc {
    const uint8_t *w;
    const uint8_t *gate;
    const float *x;
    const float *add;
    float *y;
    uint32_t rows;
    uint32_t cols;
    uint32_t item_begin;  // first work item (row tile) of this GEMV
    uint32_t pad;
};

hipError_t launch_gemv(const GemvArgs &args, hipStream_t stream);
// descs[count] plus a sentinel whose item_begin == total items.
hipError_t launch_plan(const PlanDesc *descs, uint32_t count, uint32_t items, uint32_t workgroups,
                       hipStream_t stream);
hipError_t launch_dequant(const uint8_t *w, uint32_t rows, uint32_t cols, float *out,
                          hipStream_t stream);
hipError_t launch_pack(const float *w, uint32_t rows, uint32_t cols, int algorithm, uint8_t *tiles,
                       hipStream_t stream);

// Workgroups of 256 threads the kernels are built for, and the number the
// plan kernel can keep resident per CU.
constexpr uint32_t kThreads = 256;
uint32_t plan_workgroups_per_cu();

}  // namespace q4rdna
