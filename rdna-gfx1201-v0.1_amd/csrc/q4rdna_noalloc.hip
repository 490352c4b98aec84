// q4rdna_mul_mat_ex_noalloc: q4rdna_mul_mat_ex with its split-K workspace in
// a fixed device array instead of memory the library allocates, for callers
// that cannot allocate (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).
//
// The array, `scratch`, holds Q4RDNA_NOALLOC_PARTIAL_FLOATS fp32 partial
// sums, then Q4RDNA_NOALLOC_COUNTERS arrival counters, then
// Q4RDNA_NOALLOC_SLOTS exchange slots of two-chunk launches; every GPU the
// library runs on holds its own copy until the process ends.  In host code
// the name `scratch` is only a stand-in for the symbol: the device address of
// a GPU's copy comes from hipGetSymbolAddress with that GPU current, once per
// GPU, and only that address is ever passed to a kernel.
//
// Counters and slots must be zero when a launch starts.  The array is a
// zero-initialised device variable, so both hold from the moment the code
// object is loaded, with no set-up launch (a first call captured into a graph
// or made on any stream finds them ready), and every launch leaves them so
// (the last workgroup to arrive at a row tile or 64-row block resets its
// counter; the second chunk to reach a slot puts zero back).  Partial sums
// need no clearing: every launch writes the ones it reads.  Every call on a
// GPU shares that GPU's array, so calls that overlap on one GPU race: issue
// them on one stream, or order them with events.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "q4rdna.h"
#include "q4rdna_internal.h"
#include "q4rdna_runtime.h"

namespace {

constexpr size_t kPartialBytes = static_cast<size_t>(Q4RDNA_NOALLOC_PARTIAL_FLOATS) * sizeof(float);
constexpr size_t kCounterBytes = static_cast<size_t>(Q4RDNA_NOALLOC_COUNTERS) * sizeof(uint32_t);
constexpr size_t kSlotBytes = static_cast<size_t>(Q4RDNA_NOALLOC_SLOTS) * sizeof(uint32_t);
constexpr size_t kScratchBytes = kPartialBytes + kCounterBytes + kSlotBytes;
static_assert(kPartialBytes % 256 == 0 && kCounterBytes % 256 == 0, "the counters and slots start 256-byte aligned");

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

// Device address of each GPU's copy of `scratch`, looked up on the first
// call on that GPU (a fixed table: nothing is allocated).
constexpr int kMaxDevices = 64;
std::atomic<uint8_t *> g_scratch[kMaxDevices];
std::mutex g_setup;

int scratch_of(int device, uint8_t **out) {
    if (device < 0 || device >= kMaxDevices)
        return q4rdna::set_error(Q4RDNA_ERR_ARGUMENT, "device %d is outside the no-alloc table", device);
    uint8_t *p = g_scratch[device].load(std::memory_order_acquire);
    if (p == nullptr) {
        std::lock_guard<std::mutex> lock(g_setup);
        p = g_scratch[device].load(std::memory_order_relaxed);
        if (p == nullptr) {
            // The weight's device is the current device (checked by the
            // caller), so this is that GPU's copy.
            hipError_t e = hipGetSymbolAddress(reinterpret_cast<void **>(&p), HIP_SYMBOL(scratch));
            if (e != hipSuccess || p == nullptr)
                return q4rdna::set_error(Q4RDNA_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
            g_scratch[device].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return Q4RDNA_OK;
}

}  // namespace

extern "C" int q4rdna_mul_mat_ex_noalloc(const q4rdna_weight *w, const q4rdna_weight *gate, const float *x,
                                         const float *add, float *y, const q4rdna_launch_options *options,
                                         void *stream) {
    q4rdna::TensorLaunch L{};
    int rc = q4rdna::check_mul_mat_ex(w, gate, x, add, y, options, &L);
    if (rc != Q4RDNA_OK) return rc;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const uint8_t *gt = gate ? gate->tiles : nullptr;
    if (L.partial_floats == 0 && L.counters == 0 && L.slots == 0) {
        if ((rc = q4rdna::launch_tensor_in(L, w, gt, x, add, y, nullptr, nullptr, nullptr, s)) == Q4RDNA_OK)
            q4rdna::count_gemv_launch(w->tiles, gt);
        return rc;
    }
    if (L.partial_floats > Q4RDNA_NOALLOC_PARTIAL_FLOATS || L.counters > Q4RDNA_NOALLOC_COUNTERS ||
        L.slots > Q4RDNA_NOALLOC_SLOTS)
        return q4rdna::set_error(Q4RDNA_ERR_ARGUMENT,
                                 "%ux%u needs %zu partial floats, %zu counters and %zu slots; the no-alloc scratch "
                                 "holds %u, %u and %u",
                                 w->rows, w->columns, L.partial_floats, L.counters, L.slots,
                                 static_cast<unsigned>(Q4RDNA_NOALLOC_PARTIAL_FLOATS),
                                 static_cast<unsigned>(Q4RDNA_NOALLOC_COUNTERS),
                                 static_cast<unsigned>(Q4RDNA_NOALLOC_SLOTS));
    uint8_t *base = nullptr;
    if ((rc = scratch_of(w->device, &base)) != Q4RDNA_OK) return rc;
    rc = q4rdna::launch_tensor_in(L, w, gt, x, add, y, reinterpret_cast<float *>(base),
                                  reinterpret_cast<uint32_t *>(base + kPartialBytes),
                                  reinterpret_cast<uint32_t *>(base + kPartialBytes + kCounterBytes), s);
    if (rc == Q4RDNA_OK) q4rdna::count_gemv_launch(w->tiles, gt);
    return rc;
}
