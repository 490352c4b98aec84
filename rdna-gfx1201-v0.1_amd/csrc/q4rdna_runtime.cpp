// Host runtime of the Q4_RDNA dequant-GEMV C ABI (include/q4rdna.h): sidecar
// parsing and upload, the name registry, shape policy, split-K workspaces and
// the entry points.  All compute runs in the gfx950 kernels of
// q4rdna_kernels.hip and q4rdna_mfma.hip; this file never computes a result
// on the CPU.
#include "q4rdna.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "q4rdna_host.h"
#include "q4rdna_internal.h"
#include "q4rdna_runtime.h"

namespace {
thread_local std::string g_last_error;
}  // namespace

namespace q4rdna {

int set_error(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

}  // namespace q4rdna

namespace {

using q4rdna::kGroup;
using q4rdna::kGroupChunkGroups;
using q4rdna::kTileBytes;
using q4rdna::kTileRows;
using q4rdna::set_error;
using q4rdna::host::Entry;
using q4rdna::host::FileEntry;
using q4rdna::host::FileHeader;
using q4rdna::host::kMaxSplit;
using q4rdna::host::valid_shape;

int hip_fail(hipError_t e, const char *what) {
    return set_error(Q4RDNA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int host_status(int rc, const std::string &error) {
    if (rc != Q4RDNA_OK) set_error(rc, "%s", error.c_str());
    return rc;
}

// Restores the calling thread's current device on scope exit.
class DeviceGuard {
public:
    explicit DeviceGuard(int device) {
        if (hipGetDevice(&saved_) != hipSuccess) saved_ = -1;
        if (saved_ != device) ok_ = hipSetDevice(device) == hipSuccess;
    }
    ~DeviceGuard() {
        if (saved_ >= 0) (void)hipSetDevice(saved_);
    }
    bool ok() const { return ok_; }

private:
    int saved_ = -1;
    bool ok_ = true;
};

int current_device() {
    int d = -1;
    if (hipGetDevice(&d) != hipSuccess) return -1;
    return d;
}

// Compute units per device, looked up once (a fixed table: the lookup
// allocates nothing, so allocation-free entry points may use it).
constexpr int kMaxDevices = 64;
std::atomic<uint32_t> g_cus[kMaxDevices];

uint32_t cu_count(int device) {
    if (device < 0 || device >= kMaxDevices) return 256;
    uint32_t n = g_cus[device].load(std::memory_order_relaxed);
    if (n != 0) return n;
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || v <= 0) v = 256;
    g_cus[device].store(static_cast<uint32_t>(v), std::memory_order_relaxed);
    return static_cast<uint32_t>(v);
}

int parse_index(const uint8_t *image, uint64_t image_size, uint64_t file_size, FileHeader *header,
                std::vector<Entry> *entries) {
    std::string error;
    return host_status(q4rdna::host::parse_index(image, image_size, file_size, header, entries, &error), error);
}

// Split-K exchange slots per (device, stream), kept zero between launches by
// the kernels.
struct Workspace {
    uint32_t *slots = nullptr;
    size_t slot_count = 0;
};

std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;
// Outgrown workspaces are kept, never freed: launches still queued and HIP
// graphs captured earlier keep using their pointers.  A workspace at least
// doubles when it grows, so few are ever retired.
std::vector<Workspace> g_ws_retired;

int get_workspace(int device, hipStream_t stream, size_t slots, Workspace **out) {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    Workspace &ws = g_ws[{device, stream}];
    if (ws.slot_count < slots) {
        const size_t sc = std::max(slots, 2 * ws.slot_count);
        if (ws.slots != nullptr) {
            g_ws_retired.push_back(ws);
            ws = Workspace{};
        }
        uint32_t *sl = nullptr;
        hipError_t e = hipMalloc(&sl, sc * sizeof(uint32_t));
        if (e != hipSuccess) return set_error(Q4RDNA_ERR_MEMORY, "split-K workspace: %s", hipGetErrorString(e));
        // Set once, complete before any launch uses them (launches on
        // non-blocking streams are not ordered after the null stream).
        e = hipMemset(sl, 0, sc * sizeof(uint32_t));
        if (e == hipSuccess) e = hipDeviceSynchronize();
        if (e != hipSuccess) {
            (void)hipFree(sl);
            return hip_fail(e, "hipMemset");
        }
        ws.slots = sl;
        ws.slot_count = sc;
    }
    *out = &ws;
    return Q4RDNA_OK;
}

// The clock build's record slot for the next single-launch GEMV (0 in the
// product build, which records nothing).
std::atomic<uint32_t> g_clock_launches{0};
uint32_t next_clock_slot() {
    if constexpr (!q4rdna::kSweepClocks) return 0;
    return g_clock_launches.fetch_add(1, std::memory_order_relaxed) % q4rdna::kGemvClockSlots;
}

bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

uint32_t policy_split(uint32_t rows, uint32_t cols, int device) {
    return q4rdna::host::policy_split(rows, cols, cu_count(device));
}

uint32_t resolve_split(const q4rdna_weight *w, uint32_t split) {
    if (split == 0) split = policy_split(w->rows, w->columns, w->device);
    split = std::min(split, w->columns / kGroup);
    split = std::min(split, kMaxSplit);
    return std::max<uint32_t>(split, 1);
}

// Per-tensor launch with the stream's split-K workspace.
int launch_one(const q4rdna::TensorLaunch &launch, const q4rdna_weight *w, const uint8_t *gate, const float *x,
               const float *add, float *y, hipStream_t stream) {
    uint32_t *slots = nullptr;
    if (launch.slots > 0) {
        Workspace *ws = nullptr;
        int rc = get_workspace(w->device, stream, launch.slots, &ws);
        if (rc != Q4RDNA_OK) return rc;
        slots = ws->slots;
    }
    return q4rdna::launch_tensor_in(launch, w, gate, x, add, y, slots, stream);
}

// Preconditions shared by the GEMV entry points.  NOT_APPLICABLE mirrors the
// reference's `return false` (source/q4rdna.cu:718-733,753-758,776-783).
int check_weight(const q4rdna_weight *w) {
    if (w == nullptr || w->tiles == nullptr) return set_error(Q4RDNA_NOT_APPLICABLE, "no weight");
    if (!valid_shape(w->rows, w->columns)) return set_error(Q4RDNA_ERR_ARGUMENT, "invalid weight shape %ux%u", w->rows, w->columns);
    if (!aligned(w->tiles, 16)) return set_error(Q4RDNA_ERR_ARGUMENT, "weight tiles must be 16-byte aligned");
    if (current_device() != w->device)
        return set_error(Q4RDNA_NOT_APPLICABLE, "weight lives on device %d, current device is %d", w->device, current_device());
    return Q4RDNA_OK;
}

int check_io(const float *x, const float *y) {
    if (x == nullptr || y == nullptr) return set_error(Q4RDNA_ERR_ARGUMENT, "NULL activation or output");
    if (!aligned(x, 4) || !aligned(y, 4)) return set_error(Q4RDNA_ERR_ARGUMENT, "activation/output must be 4-byte aligned");
    return Q4RDNA_OK;
}

// The kernels read x while other workgroups write y, so the two may not
// share memory; add may be y itself (each row's add is read by the thread
// that writes that row) but may not overlap it otherwise.  Sizes in floats.
int check_overlap(const float *x, size_t nx, const float *y, size_t ny, const float *add) {
    const uintptr_t x0 = reinterpret_cast<uintptr_t>(x), y0 = reinterpret_cast<uintptr_t>(y);
    if (y0 < x0 + 4 * nx && x0 < y0 + 4 * ny) return set_error(Q4RDNA_ERR_ARGUMENT, "y overlaps x");
    if (add != nullptr && add != y) {
        const uintptr_t a0 = reinterpret_cast<uintptr_t>(add);
        if (a0 < y0 + 4 * ny && y0 < a0 + 4 * ny) return set_error(Q4RDNA_ERR_ARGUMENT, "add overlaps y without being y");
    }
    return Q4RDNA_OK;
}

// Launch options beyond split_k: the kernel is the VALU kernel (0 = the
// policy, which is that kernel) and the reserved words are zero.
int check_options(const q4rdna_launch_options *options) {
    if (options == nullptr) return Q4RDNA_OK;
    if (options->kernel != Q4RDNA_KERNEL_POLICY && options->kernel != Q4RDNA_KERNEL_VALU &&
        options->kernel != Q4RDNA_KERNEL_SEQUENTIAL)
        return set_error(Q4RDNA_ERR_ARGUMENT, "unknown kernel %u", options->kernel);
    for (uint32_t r : options->reserved)
        if (r != 0) return set_error(Q4RDNA_ERR_ARGUMENT, "reserved launch options must be zero");
    return Q4RDNA_OK;
}

}  // namespace

namespace q4rdna {

int check_mul_mat_ex(const q4rdna_weight *w, const q4rdna_weight *gate, const float *x, const float *add,
                     const float *y, const q4rdna_launch_options *options, TensorLaunch *launch) {
    int rc = check_weight(w);
    if (rc != Q4RDNA_OK) return rc;
    if (gate != nullptr) {
        if ((rc = check_weight(gate)) != Q4RDNA_OK) return rc;
        if (gate->rows != w->rows || gate->columns != w->columns)
            return set_error(Q4RDNA_NOT_APPLICABLE, "up and gate shapes differ");
    }
    if ((rc = check_io(x, y)) != Q4RDNA_OK) return rc;
    if (add != nullptr && !aligned(add, 4)) return set_error(Q4RDNA_ERR_ARGUMENT, "misaligned add");
    if ((rc = check_overlap(x, w->columns, y, w->rows, add)) != Q4RDNA_OK) return rc;
    const uint32_t s = options ? options->split_k : 0;
    if (s > kMaxSplit) return set_error(Q4RDNA_ERR_ARGUMENT, "split_k %u exceeds %u", s, kMaxSplit);
    if ((rc = check_options(options)) != Q4RDNA_OK) return rc;
    TensorLaunch L{};
    if (options != nullptr && options->kernel == Q4RDNA_KERNEL_SEQUENTIAL) {
        // The old mapping sums each row in one thread: no K chunks.
        if (s > 1) return set_error(Q4RDNA_ERR_ARGUMENT, "the sequential kernel takes split_k 0 or 1, not %u", s);
        L.split = 1;
        L.sequential = true;
        *launch = L;
        return Q4RDNA_OK;
    }
    L.split = resolve_split(w, s);
    if (!gemv_shape_fits(w->rows / kTileRows, w->columns / kGroup, L.split))
        return set_error(Q4RDNA_ERR_ARGUMENT, "shape %ux%u at split %u is beyond the kernels' index range", w->rows,
                         w->columns, L.split);
    L.slots = static_cast<size_t>(host::exchange_nodes(L.split)) * w->rows * (gate ? 2 : 1);
    *launch = L;
    return Q4RDNA_OK;
}

int launch_tensor_in(const TensorLaunch &launch, const q4rdna_weight *w, const uint8_t *gate, const float *x,
                     const float *add, float *y, uint32_t *slots, hipStream_t stream) {
    GemvArgs args{};
    args.w = w->tiles;
    args.gate = gate;
    args.x = x;
    args.add = add;
    args.y = y;
    args.rows = w->rows;
    args.cols = w->columns;
    args.split = launch.split;
    args.split_magic = split_magic(launch.split);
    const uint64_t workgroups = static_cast<uint64_t>(w->rows / kTileRows) * launch.split;
    args.short_waves =
        gemv_waves(w->columns / kGroup, launch.split, workgroups, static_cast<uint32_t>(cu_count(w->device)));
    args.slots = slots;
    args.clock_slot = next_clock_slot();
    const hipError_t e = launch.sequential ? launch_gemv_sequential(args, stream) : launch_gemv(args, stream);
    if (e != hipSuccess) return hip_fail(e, "GEMV launch");
    return Q4RDNA_OK;
}

}  // namespace q4rdna

struct q4rdna_sidecar {
    int device = 0;
    uint8_t *data = nullptr;
    uint64_t data_offset = 0;
    uint64_t data_bytes = 0;
    std::vector<Entry> entries;
    std::unordered_map<std::string, uint32_t> by_name;
    std::vector<uint32_t> by_offset;                  // entry indices in data order
    std::unique_ptr<std::atomic<uint64_t>[]> hits;    // GEMV launches per entry
};

struct q4rdna_plan {
    int device = 0;
    std::vector<const uint8_t *> weights;  // every GEMV's tiles (and gate tiles): the launch's hits
    q4rdna::PlanDesc *descs = nullptr;  // count + 1 (sentinel)
    uint8_t *scratch = nullptr;         // activation digits, split-K partials and counters
    uint32_t *sched = nullptr;          // batched sweeps' [next item, finished workgroups], zero between launches
    uint8_t *table = nullptr;           // prep launch's group table (in scratch)
    uint32_t *deal = nullptr;           // single-vector sweeps' item deal (in scratch)
    uint32_t count = 0;
    uint32_t items = 0;
    uint32_t groups = 0;
    uint32_t workgroups = 0;
    uint32_t batch = 1;  // activation vectors per GEMV
    bool both_streams = false;  // some SwiGLU GEMV runs both weight streams in one item
};


namespace {

// Launch statistics, the reference's q4rdna_launches and per-entry hits
// (source/q4rdna.cu:57,73,706-709,742,764,789-791): every GEMV launch an
// entry point makes counts once, and each weight it streams that starts a
// sidecar entry counts a hit for that entry (a SwiGLU launch hits both).
std::atomic<uint64_t> g_launches{0};
std::mutex g_stats_mutex;
std::vector<q4rdna_sidecar *> g_open;  // sidecars whose entries count hits

void register_sidecar(q4rdna_sidecar *sc) {
    std::lock_guard<std::mutex> lock(g_stats_mutex);
    g_open.push_back(sc);
}

void unregister_sidecar(q4rdna_sidecar *sc) {
    std::lock_guard<std::mutex> lock(g_stats_mutex);
    g_open.erase(std::remove(g_open.begin(), g_open.end(), sc), g_open.end());
}

// One launch over `n` weights (null entries skipped).  No allocation, so
// the allocation-free entry point may count too.
void count_launch(const uint8_t *const *tiles, size_t n, uint64_t launches = 1) {
    g_launches.fetch_add(launches, std::memory_order_relaxed);
    std::lock_guard<std::mutex> lock(g_stats_mutex);
    for (size_t i = 0; i < n; ++i) {
        const uint8_t *t = tiles[i];
        if (t == nullptr) continue;
        for (q4rdna_sidecar *sc : g_open) {
            if (sc->data == nullptr || t < sc->data || t >= sc->data + sc->data_bytes) continue;
            const uint64_t rel = static_cast<uint64_t>(t - sc->data) + sc->data_offset;
            const auto it = std::lower_bound(sc->by_offset.begin(), sc->by_offset.end(), rel,
                                             [&](uint32_t idx, uint64_t v) { return sc->entries[idx].offset < v; });
            if (it != sc->by_offset.end() && sc->entries[*it].offset == rel)
                sc->hits[*it].fetch_add(launches, std::memory_order_relaxed);
            break;
        }
    }
}

void count_launch(const uint8_t *a, const uint8_t *b = nullptr, uint64_t launches = 1) {
    const uint8_t *t[2] = {a, b};
    count_launch(t, 2, launches);
}

void report_at_exit() { q4rdna_report_stats(); }

}  // namespace

namespace q4rdna {
void count_gemv_launch(const uint8_t *w, const uint8_t *gate) { count_launch(w, gate); }
}  // namespace q4rdna

namespace {

// Upload helper shared by open() and open_memory(): `read` fills a host
// chunk of the data region starting at a data-relative offset.
template <typename ReadFn>
int finish_open(const FileHeader &h, std::vector<Entry> &&entries, int device, ReadFn read, q4rdna_sidecar **out) {
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev)
        return set_error(Q4RDNA_ERR_ARGUMENT, "device %d is not available", device);
    DeviceGuard guard(device);
    if (!guard.ok()) return set_error(Q4RDNA_ERR_HIP, "hipSetDevice(%d) failed", device);
    auto sc = std::make_unique<q4rdna_sidecar>();
    sc->device = device;
    sc->data_offset = h.data_offset;
    sc->data_bytes = h.data_bytes;
    if (h.data_bytes > 0) {
        hipError_t e = hipMalloc(&sc->data, h.data_bytes);
        if (e != hipSuccess) return set_error(Q4RDNA_ERR_MEMORY, "sidecar upload: %s", hipGetErrorString(e));
        constexpr size_t kChunk = 64u << 20;  // source/q4rdna.cu:160
        std::vector<uint8_t> host(std::min<uint64_t>(kChunk, h.data_bytes));
        for (uint64_t copied = 0; copied < h.data_bytes;) {
            const size_t n = static_cast<size_t>(std::min<uint64_t>(kChunk, h.data_bytes - copied));
            if (!read(copied, host.data(), n)) {
                (void)hipFree(sc->data);
                return set_error(Q4RDNA_ERR_FORMAT, "truncated sidecar data");
            }
            e = hipMemcpy(sc->data + copied, host.data(), n, hipMemcpyHostToDevice);
            if (e != hipSuccess) {
                (void)hipFree(sc->data);
                return hip_fail(e, "sidecar upload");
            }
            copied += n;
        }
    }
    sc->entries = std::move(entries);
    for (uint32_t i = 0; i < sc->entries.size(); ++i) sc->by_name.emplace(sc->entries[i].name, i);
    sc->by_offset.resize(sc->entries.size());
    for (uint32_t i = 0; i < sc->entries.size(); ++i) sc->by_offset[i] = i;
    std::sort(sc->by_offset.begin(), sc->by_offset.end(),
              [&](uint32_t a, uint32_t b) { return sc->entries[a].offset < sc->entries[b].offset; });
    sc->hits.reset(new std::atomic<uint64_t>[sc->entries.size()]());
    register_sidecar(sc.get());
    *out = sc.release();
    return Q4RDNA_OK;
}

}  // namespace

extern "C" {

int q4rdna_abi_version(void) { return Q4RDNA_ABI_VERSION; }

const char *q4rdna_last_error(void) { return g_last_error.c_str(); }

int q4rdna_sidecar_inspect(const void *image, uint64_t image_size, uint64_t file_size, uint32_t *count) {
    FileHeader h;
    int rc = parse_index(static_cast<const uint8_t *>(image), image_size, file_size, &h, nullptr);
    if (rc != Q4RDNA_OK) return rc;
    if (count) *count = h.count;
    return Q4RDNA_OK;
}

int q4rdna_sidecar_open(const char *path, int device, q4rdna_sidecar **out) {
    if (path == nullptr || out == nullptr) return set_error(Q4RDNA_ERR_ARGUMENT, "NULL path or handle");
    *out = nullptr;
    std::ifstream in(path, std::ios::binary | std::ios::ate);
    if (!in) return set_error(Q4RDNA_ERR_IO, "cannot open %s", path);
    const uint64_t file_size = static_cast<uint64_t>(in.tellg());
    std::vector<uint8_t> head(std::min<uint64_t>(file_size, sizeof(FileHeader)));
    in.seekg(0);
    if (!in.read(reinterpret_cast<char *>(head.data()), static_cast<std::streamsize>(head.size())))
        return set_error(Q4RDNA_ERR_IO, "cannot read %s", path);
    FileHeader h{};
    if (head.size() == sizeof(FileHeader)) std::memcpy(&h, head.data(), sizeof(h));
    const uint64_t index_end = sizeof(FileHeader) + static_cast<uint64_t>(h.count) * sizeof(FileEntry);
    std::vector<uint8_t> image(static_cast<size_t>(std::min(index_end, file_size)));
    in.seekg(0);
    if (!in.read(reinterpret_cast<char *>(image.data()), static_cast<std::streamsize>(image.size())))
        return set_error(Q4RDNA_ERR_IO, "cannot read %s", path);
    std::vector<Entry> entries;
    int rc = parse_index(image.data(), image.size(), file_size, &h, &entries);
    if (rc != Q4RDNA_OK) return rc;
    auto read = [&in, &h](uint64_t rel, uint8_t *dst, size_t n) {
        in.seekg(static_cast<std::streamoff>(h.data_offset + rel));
        return static_cast<bool>(in.read(reinterpret_cast<char *>(dst), static_cast<std::streamsize>(n)));
    };
    return finish_open(h, std::move(entries), device, read, out);
}

int q4rdna_sidecar_open_memory(const void *image, uint64_t size, int device, q4rdna_sidecar **out) {
    if (image == nullptr || out == nullptr) return set_error(Q4RDNA_ERR_ARGUMENT, "NULL image or handle");
    *out = nullptr;
    FileHeader h;
    std::vector<Entry> entries;
    const auto *bytes = static_cast<const uint8_t *>(image);
    int rc = parse_index(bytes, size, size, &h, &entries);
    if (rc != Q4RDNA_OK) return rc;
    auto read = [bytes, &h](uint64_t rel, uint8_t *dst, size_t n) {
        std::memcpy(dst, bytes + h.data_offset + rel, n);
        return true;
    };
    return finish_open(h, std::move(entries), device, read, out);
}

void q4rdna_sidecar_close(q4rdna_sidecar *sidecar) {
    if (sidecar == nullptr) return;
    unregister_sidecar(sidecar);
    if (sidecar->data != nullptr) {
        DeviceGuard guard(sidecar->device);
        (void)hipFree(sidecar->data);
    }
    delete sidecar;
}

uint32_t q4rdna_sidecar_count(const q4rdna_sidecar *sidecar) {
    return sidecar ? static_cast<uint32_t>(sidecar->entries.size()) : 0u;
}

int q4rdna_sidecar_entry(const q4rdna_sidecar *sidecar, uint32_t index, char name[64], uint32_t *rows,
                         uint32_t *columns, uint64_t *offset, uint64_t *size) {
    if (sidecar == nullptr || index >= sidecar->entries.size())
        return set_error(Q4RDNA_ERR_ARGUMENT, "entry %u out of range", index);
    const Entry &e = sidecar->entries[index];
    if (name) {
        std::memset(name, 0, 64);
        std::memcpy(name, e.name.data(), std::min<size_t>(e.name.size(), 63));
    }
    if (rows) *rows = e.rows;
    if (columns) *columns = e.columns;
    if (offset) *offset = e.offset;
    if (size) *size = e.size;
    return Q4RDNA_OK;
}

int q4rdna_find(const q4rdna_sidecar *sidecar, const char *name, int64_t ne0, int64_t ne1, q4rdna_weight *out) {
    if (sidecar == nullptr || name == nullptr || out == nullptr)
        return set_error(Q4RDNA_NOT_APPLICABLE, "no sidecar or name");
    auto it = sidecar->by_name.find(name);
    if (it == sidecar->by_name.end()) return set_error(Q4RDNA_NOT_APPLICABLE, "%s is not in the sidecar", name);
    const Entry &e = sidecar->entries[it->second];
    if (ne0 != static_cast<int64_t>(e.columns) || ne1 != static_cast<int64_t>(e.rows))
        return set_error(Q4RDNA_NOT_APPLICABLE, "shape mismatch for %s", name);
    out->tiles = sidecar->data + (e.offset - sidecar->data_offset);
    out->rows = e.rows;
    out->columns = e.columns;
    out->device = sidecar->device;
    out->reserved = 0;
    return Q4RDNA_OK;
}

int q4rdna_weight_from_device(const void *tiles, uint32_t rows, uint32_t columns, int device, q4rdna_weight *out) {
    if (tiles == nullptr || out == nullptr) return set_error(Q4RDNA_ERR_ARGUMENT, "NULL tiles or output");
    if (!valid_shape(rows, columns)) return set_error(Q4RDNA_ERR_ARGUMENT, "shape %ux%u is not 32-row x 64-column tiled", rows, columns);
    if (!aligned(tiles, 16)) return set_error(Q4RDNA_ERR_ARGUMENT, "tiles must be 16-byte aligned");
    out->tiles = static_cast<const uint8_t *>(tiles);
    out->rows = rows;
    out->columns = columns;
    out->device = device;
    out->reserved = 0;
    return Q4RDNA_OK;
}

q4rdna_sidecar *q4rdna_default_sidecar(int device) {
    static std::once_flag once;
    static q4rdna_sidecar *value = nullptr;
    std::call_once(once, [device]() {
        const char *path = std::getenv("LLAMA_Q4_RDNA_SIDECAR");
        if (path == nullptr || path[0] == '\0') return;
        q4rdna_sidecar *sc = nullptr;
        if (q4rdna_sidecar_open(path, device, &sc) != Q4RDNA_OK) {
            std::fprintf(stderr, "Q4_RDNA: %s\n", g_last_error.c_str());
            return;
        }
        std::fprintf(stderr, "Q4_RDNA: loaded %u tensors, %.2f GiB on device %d from %s\n",
                     static_cast<unsigned>(sc->entries.size()),
                     static_cast<double>(sc->data_bytes) / (1024.0 * 1024.0 * 1024.0), device, path);
        value = sc;
        // The reference reports its launches when the process exits
        // (source/q4rdna.cu:176).
        std::atexit(report_at_exit);
    });
    if (value == nullptr || value->device != device) return nullptr;
    return value;
}

int q4rdna_scope_allows(const char *scope, const char *name) {
    if (name == nullptr) return 0;
    if (scope == nullptr || scope[0] == '\0') return 1;
    if (std::strcmp(scope, "ffn") == 0 && std::strstr(name, ".ffn_") == nullptr) return 0;
    if (std::strcmp(scope, "qkv-fallback") == 0 &&
        (std::strstr(name, ".attn_q.") != nullptr || std::strstr(name, ".attn_k.") != nullptr ||
         std::strstr(name, ".attn_v.") != nullptr))
        return 0;
    if (std::strcmp(scope, "hotspot") == 0 && std::strstr(name, ".ffn_gate.") == nullptr &&
        std::strstr(name, ".ffn_up.") == nullptr)
        return 0;
    if (std::strcmp(scope, "attn") == 0 && std::strstr(name, ".attn_") == nullptr) return 0;
    return 1;
}

uint32_t q4rdna_policy_split_k(uint32_t rows, uint32_t columns, int device) {
    if (!valid_shape(rows, columns)) return 0;
    return policy_split(rows, columns, device);
}

int q4rdna_mul_mat(const q4rdna_weight *w, const float *x, int64_t x_ne0, float *y, int64_t y_ne0, void *stream) {
    int rc = check_weight(w);
    if (rc != Q4RDNA_OK) return rc;
    if (x_ne0 != static_cast<int64_t>(w->columns) || y_ne0 != static_cast<int64_t>(w->rows))
        return set_error(Q4RDNA_NOT_APPLICABLE, "shape mismatch: x %lld (K %u), y %lld (M %u)",
                    static_cast<long long>(x_ne0), w->columns, static_cast<long long>(y_ne0), w->rows);
    q4rdna::TensorLaunch L{};
    if ((rc = q4rdna::check_mul_mat_ex(w, nullptr, x, nullptr, y, nullptr, &L)) != Q4RDNA_OK) return rc;
    if ((rc = launch_one(L, w, nullptr, x, nullptr, y, static_cast<hipStream_t>(stream))) == Q4RDNA_OK)
        count_launch(w->tiles);
    return rc;
}

int q4rdna_mul_mat_add(const q4rdna_weight *w, const float *x, int64_t x_ne0, const float *add, int64_t add_ne,
                       float *y, int64_t y_ne0, void *stream) {
    int rc = check_weight(w);
    if (rc != Q4RDNA_OK) return rc;
    if (x_ne0 != static_cast<int64_t>(w->columns) || y_ne0 != static_cast<int64_t>(w->rows) ||
        add_ne != static_cast<int64_t>(w->rows))
        return set_error(Q4RDNA_NOT_APPLICABLE, "shape mismatch");
    if (add == nullptr) return set_error(Q4RDNA_ERR_ARGUMENT, "NULL add");
    q4rdna::TensorLaunch L{};
    if ((rc = q4rdna::check_mul_mat_ex(w, nullptr, x, add, y, nullptr, &L)) != Q4RDNA_OK) return rc;
    if ((rc = launch_one(L, w, nullptr, x, add, y, static_cast<hipStream_t>(stream))) == Q4RDNA_OK)
        count_launch(w->tiles);
    return rc;
}

int q4rdna_mul_mat_glu(const q4rdna_weight *up, const q4rdna_weight *gate, const float *x, int64_t x_ne0, int glu_op,
                       float *y, int64_t y_ne0, void *stream) {
    if (glu_op != Q4RDNA_GLU_SWIGLU) return set_error(Q4RDNA_NOT_APPLICABLE, "only SwiGLU is handled");
    int rc = check_weight(up);
    if (rc != Q4RDNA_OK) return rc;
    if ((rc = check_weight(gate)) != Q4RDNA_OK) return rc;
    if (up->rows != gate->rows || up->columns != gate->columns || up->device != gate->device)
        return set_error(Q4RDNA_NOT_APPLICABLE, "up and gate shapes differ");
    if (x_ne0 != static_cast<int64_t>(up->columns) || y_ne0 != static_cast<int64_t>(up->rows))
        return set_error(Q4RDNA_NOT_APPLICABLE, "shape mismatch");
    q4rdna::TensorLaunch L{};
    if ((rc = q4rdna::check_mul_mat_ex(up, gate, x, nullptr, y, nullptr, &L)) != Q4RDNA_OK) return rc;
    if ((rc = launch_one(L, up, gate->tiles, x, nullptr, y, static_cast<hipStream_t>(stream))) == Q4RDNA_OK)
        count_launch(up->tiles, gate->tiles);
    return rc;
}

int q4rdna_mul_mat_ex(const q4rdna_weight *w, const q4rdna_weight *gate, const float *x, const float *add, float *y,
                      const q4rdna_launch_options *options, void *stream) {
    q4rdna::TensorLaunch L{};
    int rc = q4rdna::check_mul_mat_ex(w, gate, x, add, y, options, &L);
    if (rc != Q4RDNA_OK) return rc;
    if ((rc = launch_one(L, w, gate ? gate->tiles : nullptr, x, add, y, static_cast<hipStream_t>(stream))) ==
        Q4RDNA_OK)
        count_launch(w->tiles, gate ? gate->tiles : nullptr);
    return rc;
}

namespace {

// A validated group on the VALU kernel: one index space of row tiles over
// all GEMVs, every K chunk at most kGroupChunkGroups groups.  The split is
// the shape policy's for the group's total rows (or the caller's), raised
// until the chunks fit.
int launch_group_valu(const q4rdna_group_desc *descs, uint32_t count, const float *x, bool glu, uint32_t split_k,
                      hipStream_t stream) {
    const uint32_t cols = descs[0].weight.columns, groups = cols / kGroup;
    const int device = descs[0].weight.device;
    uint64_t total_rows = 0;
    for (uint32_t i = 0; i < count; ++i) total_rows += descs[i].weight.rows;
    if (total_rows > 0x7fffffffull) return set_error(Q4RDNA_ERR_ARGUMENT, "group too large");
    uint32_t split = split_k != 0 ? split_k : policy_split(static_cast<uint32_t>(total_rows), cols, device);
    split = std::max(split, (groups + kGroupChunkGroups - 1) / kGroupChunkGroups);
    split = std::min(split, groups);
    if (split > kMaxSplit)
        return set_error(Q4RDNA_NOT_APPLICABLE, "K = %u needs more than %u chunks of %u groups", cols, kMaxSplit,
                         kGroupChunkGroups);
    const uint32_t tiles = static_cast<uint32_t>(total_rows / kTileRows);
    const uint64_t workgroups = static_cast<uint64_t>(tiles) * split;
    if (workgroups > 0x7fffffffull || !q4rdna::gemv_shape_fits(tiles, groups, split))
        return set_error(Q4RDNA_ERR_ARGUMENT, "group too large");
    const uint32_t streams = glu ? 2u : 1u;
    size_t slots = 0;
    for (uint32_t i = 0; i < count; ++i) {
        const uint32_t rows = descs[i].weight.rows;
        slots += static_cast<size_t>(q4rdna::host::exchange_nodes(split)) * streams * rows;
    }
    Workspace *ws = nullptr;
    int rc;
    if (split > 1 && (rc = get_workspace(device, stream, slots, &ws)) != Q4RDNA_OK) return rc;
    q4rdna::GemvGroupArgs args{};
    args.x = x;
    args.count = count;
    args.cols = cols;
    args.split = split;
    args.split_magic = q4rdna::split_magic(split);
    args.tiles = tiles;
    args.short_waves = workgroups <= 4ull * cu_count(device) ? 8u : 4u;
    args.clock_slot = next_clock_slot();
    uint32_t tile_begin = 0;
    size_t soff = 0;
    for (uint32_t i = 0; i < count; ++i) {
        const q4rdna_group_desc &d = descs[i];
        const uint32_t rows = d.weight.rows;
        args.g[i] = q4rdna::GemvGroupEntry{d.weight.tiles, d.gate_tiles, d.add, d.y,
                                           split > 1 ? ws->slots + soff : nullptr, rows, tile_begin};
        tile_begin += rows / kTileRows;
        soff += static_cast<size_t>(q4rdna::host::exchange_nodes(split)) * streams * rows;
    }
    hipError_t e = q4rdna::launch_gemv_group(args, stream);
    if (e != hipSuccess) return hip_fail(e, "group GEMV launch");
    return Q4RDNA_OK;
}

}  // namespace

int q4rdna_mul_mat_group(const q4rdna_group_desc *descs, uint32_t count, const float *x, int64_t x_ne0,
                         const q4rdna_launch_options *options, void *stream) {
    if (descs == nullptr || count == 0 || count > Q4RDNA_MAX_GROUP)
        return set_error(Q4RDNA_ERR_ARGUMENT, "group of %u GEMVs is outside 1..%d", count, Q4RDNA_MAX_GROUP);
    if (x == nullptr || !aligned(x, 4)) return set_error(Q4RDNA_ERR_ARGUMENT, "NULL or misaligned activation");
    const bool glu = descs[0].gate_tiles != nullptr;
    int rc;
    for (uint32_t i = 0; i < count; ++i) {
        const q4rdna_group_desc &d = descs[i];
        if ((rc = check_weight(&d.weight)) != Q4RDNA_OK) return rc;
        if (x_ne0 != static_cast<int64_t>(d.weight.columns))
            return set_error(Q4RDNA_NOT_APPLICABLE, "descriptor %u: x holds %lld floats, K is %u", i,
                             static_cast<long long>(x_ne0), d.weight.columns);
        if ((d.gate_tiles != nullptr) != glu)
            return set_error(Q4RDNA_ERR_ARGUMENT, "gate tiles must be given for every descriptor or for none");
        if (glu && !aligned(d.gate_tiles, 16)) return set_error(Q4RDNA_ERR_ARGUMENT, "descriptor %u: misaligned gate", i);
        if (d.y == nullptr || !aligned(d.y, 4) || (d.add != nullptr && !aligned(d.add, 4)))
            return set_error(Q4RDNA_ERR_ARGUMENT, "descriptor %u: NULL or misaligned output or add", i);
        const uintptr_t y0 = reinterpret_cast<uintptr_t>(d.y), y1 = y0 + 4ull * d.weight.rows;
        const uintptr_t x0 = reinterpret_cast<uintptr_t>(x), x1 = x0 + 4ull * d.weight.columns;
        if (y0 < x1 && x0 < y1) return set_error(Q4RDNA_ERR_ARGUMENT, "descriptor %u: y overlaps x", i);
    }
    // Workgroups of different GEMVs run unordered: an output may not overlap
    // another GEMV's output or bias.  A GEMV's own add is read, row by row,
    // by the thread that writes that row of y, so it may be y itself but may
    // not overlap it otherwise.
    for (uint32_t i = 0; i < count; ++i) {
        const uintptr_t a0 = reinterpret_cast<uintptr_t>(descs[i].y), a1 = a0 + 4ull * descs[i].weight.rows;
        for (uint32_t j = 0; j < count; ++j) {
            const uintptr_t b0 = reinterpret_cast<uintptr_t>(descs[j].y), b1 = b0 + 4ull * descs[j].weight.rows;
            if (j != i && a0 < b1 && b0 < a1)
                return set_error(Q4RDNA_ERR_ARGUMENT, "descriptors %u and %u: outputs overlap", i, j);
            if (descs[j].add == nullptr || (j == i && descs[j].add == descs[i].y)) continue;
            const uintptr_t c0 = reinterpret_cast<uintptr_t>(descs[j].add), c1 = c0 + 4ull * descs[j].weight.rows;
            if (a0 < c1 && c0 < a1) {
                if (j == i) return set_error(Q4RDNA_ERR_ARGUMENT, "descriptor %u: add overlaps y without being y", i);
                return set_error(Q4RDNA_ERR_ARGUMENT, "descriptor %u: y overlaps descriptor %u's add", i, j);
            }
        }
    }
    const uint32_t split_k = options ? options->split_k : 0;
    if (split_k > kMaxSplit) return set_error(Q4RDNA_ERR_ARGUMENT, "split_k %u exceeds %u", split_k, kMaxSplit);
    if ((rc = check_options(options)) != Q4RDNA_OK) return rc;
    if (options != nullptr && options->kernel == Q4RDNA_KERNEL_SEQUENTIAL)
        return set_error(Q4RDNA_ERR_ARGUMENT, "a group launch runs the split-K kernel, not the sequential one");
    if ((rc = launch_group_valu(descs, count, x, glu, split_k, static_cast<hipStream_t>(stream))) == Q4RDNA_OK) {
        const uint8_t *t[2 * Q4RDNA_MAX_GROUP];
        for (uint32_t i = 0; i < count; ++i) {
            t[2 * i] = descs[i].weight.tiles;
            t[2 * i + 1] = descs[i].gate_tiles;
        }
        count_launch(t, 2 * count);
    }
    return rc;
}

int q4rdna_mul_mat_batch(const q4rdna_weight *w, const q4rdna_weight *gate, const float *x, uint32_t n,
                         const float *add, float *y, const q4rdna_launch_options *options, void *stream) {
    int rc = check_weight(w);
    if (rc != Q4RDNA_OK) return rc;
    if (gate != nullptr) {
        if ((rc = check_weight(gate)) != Q4RDNA_OK) return rc;
        if (gate->rows != w->rows || gate->columns != w->columns) return set_error(Q4RDNA_NOT_APPLICABLE, "up and gate shapes differ");
    }
    if ((rc = check_io(x, y)) != Q4RDNA_OK) return rc;
    if (add != nullptr && !aligned(add, 4)) return set_error(Q4RDNA_ERR_ARGUMENT, "misaligned add");
    if (n < 1 || n > Q4RDNA_MAX_BATCH) return set_error(Q4RDNA_ERR_ARGUMENT, "batch %u is outside 1..%d", n, Q4RDNA_MAX_BATCH);
    if ((rc = check_overlap(x, static_cast<size_t>(n) * w->columns, y, static_cast<size_t>(n) * w->rows, add)) !=
        Q4RDNA_OK)
        return rc;
    uint32_t split = options ? options->split_k : 0;
    if (split > kMaxSplit) return set_error(Q4RDNA_ERR_ARGUMENT, "split_k %u exceeds %u", split, kMaxSplit);
    if ((rc = check_options(options)) != Q4RDNA_OK) return rc;
    const bool sequential = options != nullptr && options->kernel == Q4RDNA_KERNEL_SEQUENTIAL;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const uint8_t *gt = gate ? gate->tiles : nullptr;
    const uint32_t groups = w->columns / kGroup;
    // Every K chunk of the n-vector kernel fits its x stage.  Longer rows than
    // 64 such chunks, and the sequential kernel, go one launch per vector.
    const uint32_t stage = q4rdna::gemv_multi_stage_groups(n);
    const uint32_t need = (groups + stage - 1) / stage;
    if (n == 1 || sequential || need > std::min(groups, kMaxSplit)) {
        const size_t M = w->rows, K = w->columns;
        q4rdna_launch_options one{};
        one.split_k = split;
        one.kernel = options ? options->kernel : Q4RDNA_KERNEL_POLICY;
        q4rdna::TensorLaunch L{};
        if ((rc = q4rdna::check_mul_mat_ex(w, gate, x, add, y, &one, &L)) != Q4RDNA_OK) return rc;
        for (uint32_t v = 0; v < n; ++v)
            if ((rc = launch_one(L, w, gt, x + v * K, add ? add + v * M : nullptr, y + v * M, s)) != Q4RDNA_OK)
                return rc;
        count_launch(w->tiles, gt, n);
        return Q4RDNA_OK;
    }
    if (split == 0) split = policy_split(w->rows, w->columns, w->device);
    split = std::min(std::max(split, need), std::min(groups, kMaxSplit));
    q4rdna::GemvArgs args{};
    args.w = w->tiles;
    args.gate = gt;
    args.x = x;
    args.add = add;
    args.y = y;
    args.rows = w->rows;
    args.cols = w->columns;
    if (!q4rdna::gemv_shape_fits(w->rows / kTileRows, groups, split))
        return set_error(Q4RDNA_ERR_ARGUMENT, "shape %ux%u at split %u is beyond the kernels' index range", w->rows,
                         w->columns, split);
    args.split = split;
    args.split_magic = q4rdna::split_magic(split);
    args.vectors = n;
    if (split > 1) {
        Workspace *ws = nullptr;
        const size_t sc = static_cast<size_t>(q4rdna::host::exchange_nodes(split)) * n * w->rows * (gate ? 2 : 1);
        if ((rc = get_workspace(w->device, s, sc, &ws)) != Q4RDNA_OK) return rc;
        args.slots = ws->slots;
    }
    hipError_t e = q4rdna::launch_gemv_multi(args, s);
    if (e != hipSuccess) return hip_fail(e, "batched GEMV launch");
    count_launch(w->tiles, gt);
    return Q4RDNA_OK;
}

int q4rdna_plan_create(const q4rdna_gemv_desc *descs, uint32_t count, int device, q4rdna_plan **out) {
    return q4rdna_plan_create_batch(descs, count, 1, device, out);
}

int q4rdna_plan_create_batch(const q4rdna_gemv_desc *descs, uint32_t count, uint32_t n, int device,
                             q4rdna_plan **out) {
    if (out == nullptr) return set_error(Q4RDNA_ERR_ARGUMENT, "NULL plan handle");
    *out = nullptr;
    // Descriptor checks, the GEMV order, the scratch layout and the item
    // deal are host work (q4rdna_host.cpp); here they are uploaded.
    q4rdna::host::PlanLayout L;
    std::string error;
    int rc = q4rdna::host::layout_plan(descs, count, n, device, cu_count(device), &L, &error);
    if (rc != Q4RDNA_OK) return host_status(rc, error);
    DeviceGuard guard(device);
    if (!guard.ok()) return set_error(Q4RDNA_ERR_HIP, "hipSetDevice(%d) failed", device);
    auto plan = std::make_unique<q4rdna_plan>();
    plan->device = device;
    plan->batch = n;
    plan->both_streams = L.both_streams;
    plan->count = count;
    for (uint32_t i = 0; i < count; ++i) {
        plan->weights.push_back(descs[i].weight.tiles);
        if (descs[i].gate_tiles != nullptr) plan->weights.push_back(descs[i].gate_tiles);
    }
    plan->items = L.items;
    plan->groups = L.groups;
    plan->workgroups = L.workgroups;
    auto cleanup = [&plan]() {
        if (plan->descs) (void)hipFree(plan->descs);
        if (plan->scratch) (void)hipFree(plan->scratch);
        if (plan->sched) (void)hipFree(plan->sched);
    };
    hipError_t e = hipMalloc(&plan->descs, L.descs.size() * sizeof(q4rdna::PlanDesc));
    if (e == hipSuccess && L.scratch_bytes > 0) e = hipMalloc(&plan->scratch, L.scratch_bytes);
    if (e == hipSuccess) e = hipMalloc(&plan->sched, 2 * sizeof(uint32_t));
    if (e != hipSuccess) {
        cleanup();
        return set_error(Q4RDNA_ERR_MEMORY, "plan buffers: %s", hipGetErrorString(e));
    }
    for (uint32_t i = 0; i < count; ++i) {
        L.descs[i].prep = plan->scratch + L.prep_off[i];
        if (L.descs[i].per > 1) {
            L.descs[i].partial = reinterpret_cast<float *>(plan->scratch + L.tail_off + L.part_off[i]);
            L.descs[i].counters = reinterpret_cast<uint32_t *>(plan->scratch + L.tail_off + L.cnt_off[i]);
        }
    }
    plan->table = plan->scratch + L.table_off;
    plan->deal = reinterpret_cast<uint32_t *>(plan->scratch + L.deal_off);
    e = hipMemcpy(plan->descs, L.descs.data(), L.descs.size() * sizeof(q4rdna::PlanDesc), hipMemcpyHostToDevice);
    if (e == hipSuccess && L.scratch_bytes > 0) e = hipMemset(plan->scratch, 0, L.scratch_bytes);
    if (e == hipSuccess && L.groups > 0) e = hipMemcpy(plan->table, L.table.data(), L.table_bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess && !L.deal.empty())
        e = hipMemcpy(plan->deal, L.deal.data(), L.deal.size() * sizeof(uint32_t), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemset(plan->sched, 0, 2 * sizeof(uint32_t));
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        cleanup();
        return hip_fail(e, "plan upload");
    }
    *out = plan.release();
    return Q4RDNA_OK;
}

namespace {

int plan_check(const q4rdna_plan *plan) {
    if (plan == nullptr) return set_error(Q4RDNA_ERR_ARGUMENT, "NULL plan");
    if (current_device() != plan->device)
        return set_error(Q4RDNA_NOT_APPLICABLE, "plan lives on device %d, current device is %d", plan->device, current_device());
    return Q4RDNA_OK;
}

}  // namespace

int q4rdna_plan_prepare(q4rdna_plan *plan, void *stream) {
    int rc = plan_check(plan);
    if (rc != Q4RDNA_OK) return rc;
    hipError_t e = plan->batch == 1
                       ? q4rdna::launch_prep(reinterpret_cast<const float *const *>(plan->table), plan->scratch,
                                             plan->groups, static_cast<hipStream_t>(stream))
                       : q4rdna::launch_prep_batch(plan->descs, reinterpret_cast<const uint32_t *>(plan->table),
                                                   plan->groups, plan->batch,
                                                   static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "plan prepare launch");
    return Q4RDNA_OK;
}

int q4rdna_plan_sweep(q4rdna_plan *plan, void *stream) {
    int rc = plan_check(plan);
    if (rc != Q4RDNA_OK) return rc;
    if (plan->items == 0) return Q4RDNA_OK;
    hipError_t e = plan->batch == 1
                       ? q4rdna::launch_plan(plan->descs, plan->deal, plan->workgroups, plan->both_streams,
                                             static_cast<hipStream_t>(stream))
                       : q4rdna::launch_plan_batch(plan->descs, plan->items, plan->batch, plan->workgroups,
                                                   plan->sched, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "plan sweep launch");
    count_launch(plan->weights.data(), plan->weights.size());
    return Q4RDNA_OK;
}

int q4rdna_plan_launch(q4rdna_plan *plan, void *stream) {
    int rc = q4rdna_plan_prepare(plan, stream);
    if (rc != Q4RDNA_OK) return rc;
    return q4rdna_plan_sweep(plan, stream);
}

void q4rdna_plan_destroy(q4rdna_plan *plan) {
    if (plan == nullptr) return;
    DeviceGuard guard(plan->device);
    if (plan->descs != nullptr) (void)hipFree(plan->descs);
    if (plan->scratch != nullptr) (void)hipFree(plan->scratch);
    if (plan->sched != nullptr) (void)hipFree(plan->sched);
    delete plan;
}

uint32_t q4rdna_plan_workgroups(const q4rdna_plan *plan) { return plan ? plan->workgroups : 0u; }

uint64_t q4rdna_launch_count(void) { return g_launches.load(std::memory_order_relaxed); }

uint64_t q4rdna_sidecar_hits(const q4rdna_sidecar *sidecar, uint32_t index) {
    if (sidecar == nullptr || index >= sidecar->entries.size()) return 0;
    return sidecar->hits[index].load(std::memory_order_relaxed);
}

// The reference's report (source/q4rdna.cu:75-112), in its words and
// shape buckets, over the entries of every open sidecar in data order.
void q4rdna_report_stats(void) {
    const uint64_t launches = g_launches.load(std::memory_order_relaxed);
    if (launches != 0)
        std::fprintf(stderr, "Q4_RDNA: launched %llu decode GEMV kernels\n", static_cast<unsigned long long>(launches));
    const bool trace = std::getenv("LLAMA_Q4_RDNA_TRACE") != nullptr;
    uint64_t s12288_4096 = 0, s4096_12288 = 0, s4096_4096 = 0, s1024_4096 = 0, other = 0;
    uint32_t unique = 0;
    std::lock_guard<std::mutex> lock(g_stats_mutex);
    for (const q4rdna_sidecar *sc : g_open) {
        for (uint32_t idx : sc->by_offset) {
            const Entry &e = sc->entries[idx];
            const uint64_t hits = sc->hits[idx].load(std::memory_order_relaxed);
            if (hits == 0) continue;
            ++unique;
            if (e.rows == 12288 && e.columns == 4096) s12288_4096 += hits;
            else if (e.rows == 4096 && e.columns == 12288) s4096_12288 += hits;
            else if (e.rows == 4096 && e.columns == 4096) s4096_4096 += hits;
            else if (e.rows == 1024 && e.columns == 4096) s1024_4096 += hits;
            else other += hits;
            if (trace)
                std::fprintf(stderr, "Q4_RDNA: hit %-31s %llu\n", e.name.c_str(), static_cast<unsigned long long>(hits));
        }
    }
    std::fprintf(stderr,
                 "Q4_RDNA: unique=%u, hits by rows x columns: 12288x4096=%llu, 4096x12288=%llu, "
                 "4096x4096=%llu, 1024x4096=%llu, other=%llu\n",
                 unique, static_cast<unsigned long long>(s12288_4096), static_cast<unsigned long long>(s4096_12288),
                 static_cast<unsigned long long>(s4096_4096), static_cast<unsigned long long>(s1024_4096),
                 static_cast<unsigned long long>(other));
}

int q4rdna_pack(const float *w, uint32_t rows, uint32_t columns, int algorithm, uint8_t *tiles, void *stream) {
    if (w == nullptr || tiles == nullptr) return set_error(Q4RDNA_ERR_ARGUMENT, "NULL input or output");
    if (!valid_shape(rows, columns)) return set_error(Q4RDNA_ERR_ARGUMENT, "shape %ux%u is not 32-row x 64-column tiled", rows, columns);
    if (algorithm < Q4RDNA_ALGO_SIDECAR || algorithm > Q4RDNA_ALGO_MSE) return set_error(Q4RDNA_ERR_ARGUMENT, "unknown algorithm %d", algorithm);
    if (!aligned(w, 16)) return set_error(Q4RDNA_ERR_ARGUMENT, "weights must be 16-byte aligned");
    hipError_t e = q4rdna::launch_pack(w, rows, columns, algorithm, tiles, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "pack launch");
    return Q4RDNA_OK;
}

int q4rdna_dequantize(const q4rdna_weight *w, float *out, void *stream) {
    int rc = check_weight(w);
    if (rc != Q4RDNA_OK) return rc;
    if (out == nullptr || !aligned(out, 4)) return set_error(Q4RDNA_ERR_ARGUMENT, "NULL or misaligned output");
    hipError_t e = q4rdna::launch_dequant(w->tiles, w->rows, w->columns, out, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "dequant launch");
    return Q4RDNA_OK;
}

}  // extern "C"

#if defined(Q4RDNA_SWEEP_CLOCKS)
// Clock build only: the record slot the next single-launch GEMV will take
// (launches take slots in order, modulo kGemvClockSlots).
extern "C" uint32_t q4rdna_gemv_clock_next(void) {
    return g_clock_launches.load(std::memory_order_relaxed) % q4rdna::kGemvClockSlots;
}
#endif
