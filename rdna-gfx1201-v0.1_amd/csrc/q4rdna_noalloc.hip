// q4rdna_mul_mat_ex_noalloc: q4rdna_mul_mat_ex with its split-K exchange
// slots in a fixed device array instead of memory the library allocates, for
// callers that cannot allocate (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc).
//
// The array, `scratch`, holds Q4RDNA_NOALLOC_SLOTS 32-bit exchange slots;
// every GPU the library runs on holds its own copy until the process ends.
// In host code the name `scratch` is only a stand-in for the symbol: the
// device address of a GPU's copy comes from hipGetSymbolAddress with that GPU
// current, once per GPU, and only that address is ever passed to a kernel.
//
// Slots must be zero when a launch starts.  The array is a zero-initialised
// device variable, so they are from the moment the code object is loaded,
// with no set-up launch (a first call captured into a graph or made on any
// stream finds them ready), and every launch leaves them so (the second
// chunk to reach a slot puts zero back).  Every call on a GPU shares that
// GPU's array, so calls that overlap on one GPU race: issue them on one
// stream, or order them with events.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "q4rdna.h"
#include "q4rdna_internal.h"
#include "q4rdna_runtime.h"

namespace {

constexpr size_t kScratchBytes = static_cast<size_t>(Q4RDNA_NOALLOC_SLOTS) * sizeof(uint32_t);

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
    if (L.slots == 0) {
        if ((rc = q4rdna::launch_tensor_in(L, w, gt, x, add, y, nullptr, s)) == Q4RDNA_OK)
            q4rdna::count_gemv_launch(w->tiles, gt);
        return rc;
    }
    if (L.slots > Q4RDNA_NOALLOC_SLOTS)
        return q4rdna::set_error(Q4RDNA_ERR_ARGUMENT,
                                 "%ux%u at split %u needs %zu exchange slots; the no-alloc scratch holds %u", w->rows,
                                 w->columns, L.split, L.slots, static_cast<unsigned>(Q4RDNA_NOALLOC_SLOTS));
    uint8_t *base = nullptr;
    if ((rc = scratch_of(w->device, &base)) != Q4RDNA_OK) return rc;
    rc = q4rdna::launch_tensor_in(L, w, gt, x, add, y, reinterpret_cast<uint32_t *>(base), s);
    if (rc == Q4RDNA_OK) q4rdna::count_gemv_launch(w->tiles, gt);
    return rc;
}
