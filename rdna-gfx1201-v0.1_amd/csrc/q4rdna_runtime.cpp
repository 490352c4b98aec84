// Host runtime of the Q4_RDNA dequant-GEMV C ABI (include/q4rdna.h): sidecar
// parsing and upload, the name registry, shape policy, split-K workspaces and
// the entry points.  All compute runs in the gfx950 kernels of
// q4rdna_kernels.hip and q4rdna_mfma.hip; this file never computes a result
// on the CPU.
#include "q4rdna.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <queue>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "q4rdna_internal.h"

namespace {

using q4rdna::kGroup;
using q4rdna::kTileBytes;
using q4rdna::kTileRows;

thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(Q4RDNA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// On-disk structures, little endian (source/q4rdna.cu:26-50).
#pragma pack(push, 1)
struct FileHeader {
    char magic[8];
    uint32_t version;
    uint32_t count;
    uint32_t group;
    uint32_t tile_rows;
    uint32_t tile_bytes;
    uint32_t reserved;
    uint64_t data_offset;
    uint64_t data_bytes;
};
struct FileEntry {
    char name[64];
    uint32_t rows;
    uint32_t columns;
    uint64_t offset;
    uint64_t size;
    uint64_t reserved;
};
#pragma pack(pop)
static_assert(sizeof(FileHeader) == 48, "sidecar header is 48 bytes");
static_assert(sizeof(FileEntry) == 96, "sidecar entry is 96 bytes");

struct Entry {
    std::string name;
    uint32_t rows;
    uint32_t columns;
    uint64_t offset;
    uint64_t size;
};

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

uint32_t cu_count(int device) {
    static std::mutex mu;
    static std::map<int, uint32_t> cache;
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(device);
    if (it != cache.end()) return it->second;
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || n <= 0) n = 256;
    cache[device] = static_cast<uint32_t>(n);
    return static_cast<uint32_t>(n);
}

// Parse and validate a header + index (loader rules of source/q4rdna.cu:129-155
// and the data-length check of :163-170).
int parse_index(const uint8_t *image, uint64_t image_size, uint64_t file_size, FileHeader *header,
                std::vector<Entry> *entries) {
    if (image == nullptr) return fail(Q4RDNA_ERR_ARGUMENT, "sidecar image is NULL");
    if (image_size < sizeof(FileHeader) || file_size < sizeof(FileHeader))
        return fail(Q4RDNA_ERR_FORMAT, "invalid sidecar header: truncated");
    FileHeader h;
    std::memcpy(&h, image, sizeof(h));
    if (std::memcmp(h.magic, "Q4RDNA1", 8) != 0 || h.version != 1 || h.group != kGroup ||
        h.tile_rows != kTileRows || h.tile_bytes != kTileBytes)
        return fail(Q4RDNA_ERR_FORMAT, "invalid sidecar header");
    const uint64_t index_end = sizeof(FileHeader) + static_cast<uint64_t>(h.count) * sizeof(FileEntry);
    if (file_size < index_end) return fail(Q4RDNA_ERR_FORMAT, "truncated sidecar index");
    if (image_size < index_end)
        return fail(Q4RDNA_ERR_ARGUMENT, "image holds %llu bytes, the index ends at %llu",
                    static_cast<unsigned long long>(image_size), static_cast<unsigned long long>(index_end));
    std::vector<Entry> out;
    out.reserve(h.count);
    for (uint32_t i = 0; i < h.count; ++i) {
        FileEntry e;
        std::memcpy(&e, image + sizeof(FileHeader) + static_cast<uint64_t>(i) * sizeof(FileEntry), sizeof(e));
        if (std::memchr(e.name, '\0', sizeof(e.name)) == nullptr || e.offset < h.data_offset ||
            e.offset + e.size < e.offset || e.offset + e.size > h.data_offset + h.data_bytes ||
            e.rows % kTileRows != 0 || e.columns % kGroup != 0 ||
            e.size != static_cast<uint64_t>(e.rows) * e.columns * 34 / kGroup)
            return fail(Q4RDNA_ERR_FORMAT, "invalid sidecar entry %u", i);
        out.push_back(Entry{std::string(e.name), e.rows, e.columns, e.offset, e.size});
    }
    if (h.data_offset > file_size || h.data_bytes > file_size - h.data_offset)
        return fail(Q4RDNA_ERR_FORMAT, "truncated sidecar data");
    if (header) *header = h;
    if (entries) *entries = std::move(out);
    return Q4RDNA_OK;
}

// Split-K scratch per (device, stream): partial sums and per-row-tile
// arrival counters (kept zero between launches by the kernel itself).
struct Workspace {
    float *partial = nullptr;
    uint32_t *counters = nullptr;
    size_t partial_floats = 0;
    size_t counter_count = 0;
};

std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;
// Outgrown workspaces are kept, never freed: launches still queued and HIP
// graphs captured earlier keep using their pointers.  A workspace at least
// doubles when it grows, so few are ever retired.
std::vector<Workspace> g_ws_retired;

int get_workspace(int device, hipStream_t stream, size_t partial_floats, size_t counters, Workspace **out) {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    Workspace &ws = g_ws[{device, stream}];
    if (ws.partial_floats < partial_floats || ws.counter_count < counters) {
        const size_t pf = std::max(partial_floats, 2 * ws.partial_floats);
        const size_t cc = std::max(counters, 2 * ws.counter_count);
        if (ws.partial != nullptr || ws.counters != nullptr) {
            g_ws_retired.push_back(ws);
            ws = Workspace{};
        }
        float *p = nullptr;
        uint32_t *c = nullptr;
        hipError_t e = hipMalloc(&p, pf * sizeof(float));
        if (e != hipSuccess) return fail(Q4RDNA_ERR_MEMORY, "split-K workspace: %s", hipGetErrorString(e));
        e = hipMalloc(&c, cc * sizeof(uint32_t));
        if (e != hipSuccess) {
            (void)hipFree(p);
            return fail(Q4RDNA_ERR_MEMORY, "split-K counters: %s", hipGetErrorString(e));
        }
        // Zeroed once, complete before any launch uses them (launches on
        // non-blocking streams are not ordered after the null stream).
        e = hipMemset(c, 0, cc * sizeof(uint32_t));
        if (e == hipSuccess) e = hipDeviceSynchronize();
        if (e != hipSuccess) {
            (void)hipFree(p);
            (void)hipFree(c);
            return hip_fail(e, "hipMemset");
        }
        ws.partial = p;
        ws.counters = c;
        ws.partial_floats = pf;
        ws.counter_count = cc;
    }
    *out = &ws;
    return Q4RDNA_OK;
}

bool valid_shape(uint32_t rows, uint32_t cols) {
    return rows > 0 && cols > 0 && rows % kTileRows == 0 && cols % kGroup == 0;
}

bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

constexpr uint32_t kMaxSplit = 64;

uint32_t policy_split(uint32_t rows, uint32_t cols, int device) {
    // About 32 groups per workgroup (eight waves of four tiles, all in flight
    // at once) and at most 8 chunks; more chunks only when the row tiles are
    // so few that under a quarter of the CUs would get a workgroup, fewer
    // when there would be more than six workgroups per CU.  Measured on
    // MI355X (split sweep, with and without a SwiGLU gate): 4096x4096 best at
    // 2, 1024x4096 at 2-4, 12288x4096 at 2, 4096x12288 at 6, 2048x28672 at
    // 7-8, 151936x4096 at 1-2.
    const uint32_t tiles = rows / kTileRows;
    const uint32_t groups = cols / kGroup;
    const uint32_t cus = cu_count(device);
    uint32_t split = std::min<uint32_t>((groups + 31) / 32, 8);
    if (static_cast<uint64_t>(tiles) * split * 4 < cus)
        split = std::min((cus / 4 + tiles - 1) / tiles, std::max<uint32_t>(1, groups / 16));
    if (static_cast<uint64_t>(tiles) * split > 6ull * cus) split = std::max<uint32_t>(1, 6 * cus / tiles);
    split = std::min(split, std::min(groups, kMaxSplit));
    return std::max<uint32_t>(split, 1);
}

int launch_one(const q4rdna_weight *w, const uint8_t *gate, const float *x, const float *add, float *y,
               uint32_t split, hipStream_t stream) {
    q4rdna::GemvArgs args{};
    args.w = w->tiles;
    args.gate = gate;
    args.x = x;
    args.add = add;
    args.y = y;
    args.rows = w->rows;
    args.cols = w->columns;
    const uint32_t groups = w->columns / kGroup;
    if (split == 0) split = policy_split(w->rows, w->columns, w->device);
    split = std::min(split, groups);
    split = std::min(split, kMaxSplit);
    args.split = std::max<uint32_t>(split, 1);
    // Eight waves per workgroup while the launch is latency-bound (at most
    // four workgroups per CU); with more, four waves of up to 16 tiles keep
    // more bytes in flight per CU (151936x4096: 60 us against 68).
    const uint64_t workgroups = static_cast<uint64_t>(w->rows / kTileRows) * args.split;
    args.short_waves = workgroups <= 4ull * cu_count(w->device) ? 8u : 4u;
    if (args.split > 1) {
        Workspace *ws = nullptr;
        const size_t pf = static_cast<size_t>(args.split) * w->rows * (gate ? 2 : 1);
        int rc = get_workspace(w->device, stream, pf, w->rows / kTileRows, &ws);
        if (rc != Q4RDNA_OK) return rc;
        args.partial = ws->partial;
        args.counters = ws->counters;
    }
    hipError_t e = q4rdna::launch_gemv(args, stream);
    if (e != hipSuccess) return hip_fail(e, "GEMV launch");
    return Q4RDNA_OK;
}

// Preconditions shared by the GEMV entry points.  NOT_APPLICABLE mirrors the
// reference's `return false` (source/q4rdna.cu:718-733,753-758,776-783).
int check_weight(const q4rdna_weight *w) {
    if (w == nullptr || w->tiles == nullptr) return fail(Q4RDNA_NOT_APPLICABLE, "no weight");
    if (!valid_shape(w->rows, w->columns)) return fail(Q4RDNA_ERR_ARGUMENT, "invalid weight shape %ux%u", w->rows, w->columns);
    if (!aligned(w->tiles, 16)) return fail(Q4RDNA_ERR_ARGUMENT, "weight tiles must be 16-byte aligned");
    if (current_device() != w->device)
        return fail(Q4RDNA_NOT_APPLICABLE, "weight lives on device %d, current device is %d", w->device, current_device());
    return Q4RDNA_OK;
}

int check_io(const float *x, const float *y) {
    if (x == nullptr || y == nullptr) return fail(Q4RDNA_ERR_ARGUMENT, "NULL activation or output");
    if (!aligned(x, 4) || !aligned(y, 4)) return fail(Q4RDNA_ERR_ARGUMENT, "activation/output must be 4-byte aligned");
    return Q4RDNA_OK;
}

}  // namespace

struct q4rdna_sidecar {
    int device = 0;
    uint8_t *data = nullptr;
    uint64_t data_offset = 0;
    uint64_t data_bytes = 0;
    std::vector<Entry> entries;
    std::unordered_map<std::string, uint32_t> by_name;
};

struct q4rdna_plan {
    int device = 0;
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

// Upload helper shared by open() and open_memory(): `read` fills a host
// chunk of the data region starting at a data-relative offset.
template <typename ReadFn>
int finish_open(const FileHeader &h, std::vector<Entry> &&entries, int device, ReadFn read, q4rdna_sidecar **out) {
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev)
        return fail(Q4RDNA_ERR_ARGUMENT, "device %d is not available", device);
    DeviceGuard guard(device);
    if (!guard.ok()) return fail(Q4RDNA_ERR_HIP, "hipSetDevice(%d) failed", device);
    auto sc = std::make_unique<q4rdna_sidecar>();
    sc->device = device;
    sc->data_offset = h.data_offset;
    sc->data_bytes = h.data_bytes;
    if (h.data_bytes > 0) {
        hipError_t e = hipMalloc(&sc->data, h.data_bytes);
        if (e != hipSuccess) return fail(Q4RDNA_ERR_MEMORY, "sidecar upload: %s", hipGetErrorString(e));
        constexpr size_t kChunk = 64u << 20;  // source/q4rdna.cu:160
        std::vector<uint8_t> host(std::min<uint64_t>(kChunk, h.data_bytes));
        for (uint64_t copied = 0; copied < h.data_bytes;) {
            const size_t n = static_cast<size_t>(std::min<uint64_t>(kChunk, h.data_bytes - copied));
            if (!read(copied, host.data(), n)) {
                (void)hipFree(sc->data);
                return fail(Q4RDNA_ERR_FORMAT, "truncated sidecar data");
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
    if (path == nullptr || out == nullptr) return fail(Q4RDNA_ERR_ARGUMENT, "NULL path or handle");
    *out = nullptr;
    std::ifstream in(path, std::ios::binary | std::ios::ate);
    if (!in) return fail(Q4RDNA_ERR_IO, "cannot open %s", path);
    const uint64_t file_size = static_cast<uint64_t>(in.tellg());
    std::vector<uint8_t> head(std::min<uint64_t>(file_size, sizeof(FileHeader)));
    in.seekg(0);
    if (!in.read(reinterpret_cast<char *>(head.data()), static_cast<std::streamsize>(head.size())))
        return fail(Q4RDNA_ERR_IO, "cannot read %s", path);
    FileHeader h{};
    if (head.size() == sizeof(FileHeader)) std::memcpy(&h, head.data(), sizeof(h));
    const uint64_t index_end = sizeof(FileHeader) + static_cast<uint64_t>(h.count) * sizeof(FileEntry);
    std::vector<uint8_t> image(static_cast<size_t>(std::min(index_end, file_size)));
    in.seekg(0);
    if (!in.read(reinterpret_cast<char *>(image.data()), static_cast<std::streamsize>(image.size())))
        return fail(Q4RDNA_ERR_IO, "cannot read %s", path);
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
    if (image == nullptr || out == nullptr) return fail(Q4RDNA_ERR_ARGUMENT, "NULL image or handle");
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
        return fail(Q4RDNA_ERR_ARGUMENT, "entry %u out of range", index);
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
        return fail(Q4RDNA_NOT_APPLICABLE, "no sidecar or name");
    auto it = sidecar->by_name.find(name);
    if (it == sidecar->by_name.end()) return fail(Q4RDNA_NOT_APPLICABLE, "%s is not in the sidecar", name);
    const Entry &e = sidecar->entries[it->second];
    if (ne0 != static_cast<int64_t>(e.columns) || ne1 != static_cast<int64_t>(e.rows))
        return fail(Q4RDNA_NOT_APPLICABLE, "shape mismatch for %s", name);
    out->tiles = sidecar->data + (e.offset - sidecar->data_offset);
    out->rows = e.rows;
    out->columns = e.columns;
    out->device = sidecar->device;
    out->reserved = 0;
    return Q4RDNA_OK;
}

int q4rdna_weight_from_device(const void *tiles, uint32_t rows, uint32_t columns, int device, q4rdna_weight *out) {
    if (tiles == nullptr || out == nullptr) return fail(Q4RDNA_ERR_ARGUMENT, "NULL tiles or output");
    if (!valid_shape(rows, columns)) return fail(Q4RDNA_ERR_ARGUMENT, "shape %ux%u is not 32-row x 64-column tiled", rows, columns);
    if (!aligned(tiles, 16)) return fail(Q4RDNA_ERR_ARGUMENT, "tiles must be 16-byte aligned");
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
        return fail(Q4RDNA_NOT_APPLICABLE, "shape mismatch: x %lld (K %u), y %lld (M %u)",
                    static_cast<long long>(x_ne0), w->columns, static_cast<long long>(y_ne0), w->rows);
    if ((rc = check_io(x, y)) != Q4RDNA_OK) return rc;
    return launch_one(w, nullptr, x, nullptr, y, 0, static_cast<hipStream_t>(stream));
}

int q4rdna_mul_mat_add(const q4rdna_weight *w, const float *x, int64_t x_ne0, const float *add, int64_t add_ne,
                       float *y, int64_t y_ne0, void *stream) {
    int rc = check_weight(w);
    if (rc != Q4RDNA_OK) return rc;
    if (x_ne0 != static_cast<int64_t>(w->columns) || y_ne0 != static_cast<int64_t>(w->rows) ||
        add_ne != static_cast<int64_t>(w->rows))
        return fail(Q4RDNA_NOT_APPLICABLE, "shape mismatch");
    if ((rc = check_io(x, y)) != Q4RDNA_OK) return rc;
    if (add == nullptr || !aligned(add, 4)) return fail(Q4RDNA_ERR_ARGUMENT, "NULL or misaligned add");
    return launch_one(w, nullptr, x, add, y, 0, static_cast<hipStream_t>(stream));
}

int q4rdna_mul_mat_glu(const q4rdna_weight *up, const q4rdna_weight *gate, const float *x, int64_t x_ne0, int glu_op,
                       float *y, int64_t y_ne0, void *stream) {
    if (glu_op != Q4RDNA_GLU_SWIGLU) return fail(Q4RDNA_NOT_APPLICABLE, "only SwiGLU is handled");
    int rc = check_weight(up);
    if (rc != Q4RDNA_OK) return rc;
    if ((rc = check_weight(gate)) != Q4RDNA_OK) return rc;
    if (up->rows != gate->rows || up->columns != gate->columns || up->device != gate->device)
        return fail(Q4RDNA_NOT_APPLICABLE, "up and gate shapes differ");
    if (x_ne0 != static_cast<int64_t>(up->columns) || y_ne0 != static_cast<int64_t>(up->rows))
        return fail(Q4RDNA_NOT_APPLICABLE, "shape mismatch");
    if ((rc = check_io(x, y)) != Q4RDNA_OK) return rc;
    return launch_one(up, gate->tiles, x, nullptr, y, 0, static_cast<hipStream_t>(stream));
}

int q4rdna_mul_mat_ex(const q4rdna_weight *w, const q4rdna_weight *gate, const float *x, const float *add, float *y,
                      const q4rdna_launch_options *options, void *stream) {
    int rc = check_weight(w);
    if (rc != Q4RDNA_OK) return rc;
    if (gate != nullptr) {
        if ((rc = check_weight(gate)) != Q4RDNA_OK) return rc;
        if (gate->rows != w->rows || gate->columns != w->columns) return fail(Q4RDNA_NOT_APPLICABLE, "up and gate shapes differ");
    }
    if ((rc = check_io(x, y)) != Q4RDNA_OK) return rc;
    if (add != nullptr && !aligned(add, 4)) return fail(Q4RDNA_ERR_ARGUMENT, "misaligned add");
    const uint32_t split = options ? options->split_k : 0;
    if (split > kMaxSplit) return fail(Q4RDNA_ERR_ARGUMENT, "split_k %u exceeds %u", split, kMaxSplit);
    return launch_one(w, gate ? gate->tiles : nullptr, x, add, y, split, static_cast<hipStream_t>(stream));
}

int q4rdna_mul_mat_batch(const q4rdna_weight *w, const q4rdna_weight *gate, const float *x, uint32_t n,
                         const float *add, float *y, const q4rdna_launch_options *options, void *stream) {
    int rc = check_weight(w);
    if (rc != Q4RDNA_OK) return rc;
    if (gate != nullptr) {
        if ((rc = check_weight(gate)) != Q4RDNA_OK) return rc;
        if (gate->rows != w->rows || gate->columns != w->columns) return fail(Q4RDNA_NOT_APPLICABLE, "up and gate shapes differ");
    }
    if ((rc = check_io(x, y)) != Q4RDNA_OK) return rc;
    if (add != nullptr && !aligned(add, 4)) return fail(Q4RDNA_ERR_ARGUMENT, "misaligned add");
    if (n < 1 || n > Q4RDNA_MAX_BATCH) return fail(Q4RDNA_ERR_ARGUMENT, "batch %u is outside 1..%d", n, Q4RDNA_MAX_BATCH);
    uint32_t split = options ? options->split_k : 0;
    if (split > kMaxSplit) return fail(Q4RDNA_ERR_ARGUMENT, "split_k %u exceeds %u", split, kMaxSplit);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const uint8_t *gt = gate ? gate->tiles : nullptr;
    const uint32_t groups = w->columns / kGroup;
    // Every K chunk of the n-vector kernel fits its x stage.  Longer rows than
    // 64 such chunks go one launch per vector.
    const uint32_t stage = q4rdna::gemv_multi_stage_groups(n);
    const uint32_t need = (groups + stage - 1) / stage;
    if (n == 1 || need > std::min(groups, kMaxSplit)) {
        const size_t M = w->rows, K = w->columns;
        for (uint32_t v = 0; v < n; ++v)
            if ((rc = launch_one(w, gt, x + v * K, add ? add + v * M : nullptr, y + v * M, split, s)) != Q4RDNA_OK)
                return rc;
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
    args.split = split;
    args.vectors = n;
    if (split > 1) {
        Workspace *ws = nullptr;
        const size_t pf = static_cast<size_t>(split) * n * w->rows * (gate ? 2 : 1);
        if ((rc = get_workspace(w->device, s, pf, w->rows / kTileRows, &ws)) != Q4RDNA_OK) return rc;
        args.partial = ws->partial;
        args.counters = ws->counters;
    }
    hipError_t e = q4rdna::launch_gemv_multi(args, s);
    if (e != hipSuccess) return hip_fail(e, "batched GEMV launch");
    return Q4RDNA_OK;
}

namespace {

// Deal of a single-vector sweep's items to its workgroups.  cost[i] is item
// i's weight in the sweep (tiles streamed plus the item end); weight[b] is
// workgroup b's time per unit of cost (1024 = 1).  Items go in order,
// longest GEMV first, each to the workgroup that would finish it first;
// then moves and swaps of one item between the latest workgroup and an
// earlier one bring the latest forward while any does (each lowers the
// sorted vector of finish times, so this ends; it is capped besides).  On
// the Qwen3-8B stack (2,304 items of 192 groups x 64 rows, 9,792 of 64
// groups x 128 rows, 512 workgroups, equal weights) a round-robin deal
// leaves the most-loaded workgroup 53 units of 64 groups x 64 rows against
// a mean of 51.75; this one 52.
// Returns per workgroup the offset of its list (workgroups + 1 offsets)
// and the lists, each in increasing item order.
std::vector<uint32_t> deal_items(const std::vector<uint32_t> &cost, const std::vector<uint32_t> &weight) {
    const uint32_t workgroups = static_cast<uint32_t>(weight.size());
    std::vector<std::vector<uint32_t>> own(workgroups);
    std::vector<uint64_t> load(workgroups, 0);
    auto finish = [&](uint32_t b, uint64_t l) { return l * weight[b]; };
    // One heap of workgroups per distinct weight, least loaded on top.
    using Slot = std::pair<uint64_t, uint32_t>;
    using Heap = std::priority_queue<Slot, std::vector<Slot>, std::greater<Slot>>;
    std::map<uint32_t, Heap> lightest;
    for (uint32_t b = 0; b < workgroups; ++b) lightest[weight[b]].push({0, b});
    for (uint32_t i = 0; i < cost.size(); ++i) {
        Heap *best = nullptr;
        uint64_t best_t = UINT64_MAX;
        for (auto &kv : lightest) {
            const uint64_t t = (kv.second.top().first + cost[i]) * kv.first;
            if (t < best_t) best_t = t, best = &kv.second;
        }
        const uint32_t b = best->top().second;
        best->pop();
        own[b].push_back(i);
        load[b] += cost[i];
        best->push({load[b], b});
    }
    // One item of each distinct cost a workgroup holds (the candidates of a
    // move; which item of a cost moves does not change any load).
    auto kinds = [&](uint32_t b) {
        std::vector<uint32_t> k;
        for (uint32_t pos = 0; pos < own[b].size(); ++pos) {
            bool seen = false;
            for (uint32_t q : k) seen |= cost[own[b][q]] == cost[own[b][pos]];
            if (!seen) k.push_back(pos);
        }
        return k;
    };
    std::vector<uint32_t> by_time(workgroups);
    for (uint32_t round = 0; round < 4 * workgroups; ++round) {
        uint32_t a = 0;
        for (uint32_t b = 1; b < workgroups; ++b)
            if (finish(b, load[b]) > finish(a, load[a])) a = b;
        const uint64_t t_a = finish(a, load[a]);
        for (uint32_t b = 0; b < workgroups; ++b) by_time[b] = b;
        std::sort(by_time.begin(), by_time.end(),
                  [&](uint32_t x, uint32_t y) { return finish(x, load[x]) < finish(y, load[y]); });
        const std::vector<uint32_t> ka = kinds(a);
        uint64_t best_max = t_a;
        uint32_t best_b = 0, best_pa = 0, best_pb = 0;
        bool found = false;
        for (uint32_t b : by_time) {
            if (b == a || finish(b, load[b]) >= t_a) break;
            std::vector<uint32_t> kb = kinds(b);
            kb.push_back(UINT32_MAX);  // a move with nothing in return
            for (uint32_t pa : ka)
                for (uint32_t pb : kb) {
                    const uint64_t give = cost[own[a][pa]], take = pb == UINT32_MAX ? 0 : cost[own[b][pb]];
                    if (give <= take) continue;
                    const uint64_t m = std::max(finish(a, load[a] - (give - take)), finish(b, load[b] + (give - take)));
                    if (m < best_max) {
                        best_max = m;
                        best_b = b;
                        best_pa = pa;
                        best_pb = pb;
                        found = true;
                    }
                }
            if (found) break;
        }
        if (!found) break;
        const uint32_t item_a = own[a][best_pa];
        own[a].erase(own[a].begin() + best_pa);
        load[a] -= cost[item_a];
        if (best_pb != UINT32_MAX) {
            const uint32_t item_b = own[best_b][best_pb];
            own[best_b].erase(own[best_b].begin() + best_pb);
            load[best_b] -= cost[item_b];
            own[a].push_back(item_b);
            load[a] += cost[item_b];
        }
        own[best_b].push_back(item_a);
        load[best_b] += cost[item_a];
    }
    std::vector<uint32_t> deal(workgroups + 1 + cost.size());
    uint32_t k = 0;
    for (uint32_t b = 0; b < workgroups; ++b) {
        deal[b] = k;
        std::sort(own[b].begin(), own[b].end());
        for (uint32_t i : own[b]) deal[workgroups + 1 + k++] = i;
    }
    deal[workgroups] = k;
    return deal;
}

}  // namespace

int q4rdna_plan_create(const q4rdna_gemv_desc *descs, uint32_t count, int device, q4rdna_plan **out) {
    return q4rdna_plan_create_batch(descs, count, 1, device, out);
}

int q4rdna_plan_create_batch(const q4rdna_gemv_desc *descs, uint32_t count, uint32_t n, int device,
                             q4rdna_plan **out) {
    if (out == nullptr || (descs == nullptr && count > 0)) return fail(Q4RDNA_ERR_ARGUMENT, "NULL descriptors or handle");
    *out = nullptr;
    if (n < 1 || n > Q4RDNA_MAX_BATCH) return fail(Q4RDNA_ERR_ARGUMENT, "batch %u is outside 1..%d", n, Q4RDNA_MAX_BATCH);
    using q4rdna::kChunkGroups;
    // Single vectors: 64-row blocks, kPrepBytes per group.  Batches: 256-row
    // blocks, one kBatchQuadBytesHost record per (group, quad of vectors).
    const uint32_t block_rows = n == 1 ? q4rdna::kBlockRows : q4rdna::kBatchBlockRows;
    const uint64_t prep_per_group =
        n == 1 ? q4rdna::kPrepBytes : static_cast<uint64_t>((n + 3) / 4) * q4rdna::kBatchQuadBytesHost;
    const uint32_t chunk_groups = n == 1 ? kChunkGroups : q4rdna::kBatchChunkGroups;
    for (uint32_t i = 0; i < count; ++i) {
        const q4rdna_gemv_desc &d = descs[i];
        if (d.weight.tiles == nullptr || d.x == nullptr || d.y == nullptr)
            return fail(Q4RDNA_ERR_ARGUMENT, "descriptor %u has a NULL pointer", i);
        if (!valid_shape(d.weight.rows, d.weight.columns) || !aligned(d.weight.tiles, 16) ||
            (d.gate_tiles != nullptr && !aligned(d.gate_tiles, 16)) || !aligned(d.x, 16) || !aligned(d.y, 4) ||
            (d.add != nullptr && !aligned(d.add, 4)))
            return fail(Q4RDNA_ERR_ARGUMENT, "descriptor %u: invalid shape or alignment", i);
        if (d.weight.device != device) return fail(Q4RDNA_ERR_ARGUMENT, "descriptor %u lives on device %d", i, d.weight.device);
    }
    // The GEMVs of a plan are independent, so the sweep may take them in any
    // order: GEMVs with longer items (wider K chunks) go first, so that the
    // end of the sweep, where workgroups run out of items, deals short ones.
    std::vector<uint32_t> order(count);
    for (uint32_t i = 0; i < count; ++i) order[i] = i;
    // A single-vector SwiGLU GEMV whose rows fit one chunk runs both weight
    // streams in one item per block (no split-K partials).
    auto both_streams = [&](uint32_t i) {
        return n == 1 && descs[i].gate_tiles != nullptr && descs[i].weight.columns / kGroup <= chunk_groups;
    };
    // A single-vector GEMV with no gate whose rows fit one 64-group step
    // block runs two 64-row blocks per item: half the item ends.
    auto pairs = [&](uint32_t i) {
        return n == 1 && descs[i].gate_tiles == nullptr && descs[i].weight.columns / kGroup <= 64;
    };
    auto item_groups = [&](uint32_t i) {
        return std::min(descs[i].weight.columns / kGroup, chunk_groups) * (both_streams(i) || pairs(i) ? 2u : 1u);
    };
    std::stable_sort(order.begin(), order.end(), [&](uint32_t a, uint32_t b) { return item_groups(a) > item_groups(b); });
    std::vector<q4rdna::PlanDesc> host(static_cast<size_t>(count) + 1);
    // Scratch layout: activation digits of every group in global group order
    // (prep_per_group each), the prep launch's group table, then per GEMV
    // with several items per block its partials and per-block counters
    // (offsets below are relative to the end of the first two regions).
    // host[i] describes descs[order[i]].
    uint64_t items = 0, groups = 0, scratch = 0;
    std::vector<uint64_t> part_off(count), cnt_off(count);
    for (uint32_t i = 0; i < count; ++i) {
        const q4rdna_gemv_desc &d = descs[order[i]];
        const uint32_t g = d.weight.columns / kGroup;
        const uint32_t chunks = (g + chunk_groups - 1) / chunk_groups;
        const bool pair = pairs(order[i]);
        const uint32_t item_rows = pair ? 2 * block_rows : block_rows;
        const uint32_t blocks = (d.weight.rows + item_rows - 1) / item_rows;
        const uint32_t streams = d.gate_tiles != nullptr ? 2u : 1u;
        q4rdna::PlanDesc &p = host[i];
        p.w = d.weight.tiles;
        p.gate = d.gate_tiles;
        p.x = d.x;
        p.add = d.add;
        p.y = d.y;
        p.rows = d.weight.rows;
        p.cols = d.weight.columns;
        p.item_begin = static_cast<uint32_t>(items);
        p.group_begin = static_cast<uint32_t>(groups);
        p.chunks = chunks;
        p.streams = streams;
        p.per = both_streams(order[i]) || pair ? 1u : chunks * streams;
        p.pair = pair ? 1u : 0u;
        if (p.per > 1) {
            part_off[i] = scratch;
            scratch += static_cast<uint64_t>(chunks) * streams * n * d.weight.rows * sizeof(float);
            scratch = (scratch + 255) & ~uint64_t(255);
            cnt_off[i] = scratch;
            scratch += static_cast<uint64_t>(blocks) * sizeof(uint32_t);
        }
        scratch = (scratch + 255) & ~uint64_t(255);
        items += static_cast<uint64_t>(blocks) * p.per;
        groups += g;
        if (items > 0xffffffffull || groups * n > 0xffffffffull) return fail(Q4RDNA_ERR_ARGUMENT, "plan too large");
    }
    host[count] = q4rdna::PlanDesc{};
    host[count].item_begin = static_cast<uint32_t>(items);
    host[count].group_begin = static_cast<uint32_t>(groups);
    // Group table of the prep launch: single vectors get each group's
    // activation address (one load, no descriptor lookup); batches the
    // descriptor index of each group.
    const uint64_t table_off = (groups * prep_per_group + 255) & ~uint64_t(255);
    const uint64_t table_bytes = groups * (n == 1 ? sizeof(uint64_t) : sizeof(uint32_t));
    uint32_t per_cu = q4rdna::plan_workgroups_per_cu();
    if (const char *env = std::getenv("Q4RDNA_PLAN_WG_PER_CU")) {  // tuning sweeps only
        const int v = std::atoi(env);
        if (v >= 1 && v <= 16) per_cu = static_cast<uint32_t>(v);
    }
    const uint32_t workgroups =
        static_cast<uint32_t>(std::max<uint64_t>(1, std::min<uint64_t>(uint64_t(cu_count(device)) * per_cu, items)));
    // Single vectors: the items' deal to the workgroups, after the table.
    std::vector<uint32_t> deal;
    if (n == 1) {
        std::vector<uint32_t> cost(items);
        for (uint32_t i = 0; i < count; ++i) {
            const q4rdna::PlanDesc &p = host[i];
            const uint32_t g = p.cols / kGroup;
            for (uint32_t item = p.item_begin; item < host[i + 1].item_begin; ++item) {
                const uint32_t part = (item - p.item_begin) % p.per;
                const uint32_t chunk = part % p.chunks;
                const uint32_t chunk_g = std::min(g, (chunk + 1) * chunk_groups) - chunk * chunk_groups;
                // Pairs stream four row tiles, items of both streams two
                // per stream, other items two.
                const uint32_t row_tiles = p.pair || (p.streams > 1 && p.per == 1) ? 4u : 2u;
                cost[item] = row_tiles * chunk_g + q4rdna::kItemEndTiles;
            }
        }
        // The kernel's form: the offsets (padded to 8 bytes), then per item
        // its descriptor index and its index within the descriptor.
        // Of the two workgroups a CU holds, the one dispatched first (b <
        // CUs, as workgroups are dispatched in order) wins the CU's
        // arbitration and streams faster.  With equal loads on the Qwen3-8B
        // stack, workgroups b >= CUs finished 20 us after the others (mean
        // 526.9 against 506.4 us, per-workgroup clock reads), so the CU ran
        // its second workgroup alone at the end.  Swept on one box, a weight
        // of 1.074 for the second slot ended both together and gave the
        // shortest step (1.0 / 1.039 / 1.074 / 1.123 / 1.172: 553.6 /
        // 550.3 / 549.4 / 553.6 / 557.1 us).
        const uint32_t cus = cu_count(device);
        uint32_t second_slot = 1100;
        if (const char *env = std::getenv("Q4RDNA_PLAN_SLOT_WEIGHT")) {  // tuning sweeps only
            const int v = std::atoi(env);
            if (v >= 512 && v <= 4096) second_slot = static_cast<uint32_t>(v);
        }
        std::vector<uint32_t> weight(workgroups, 1024);
        for (uint32_t b = cus; b < workgroups; ++b) weight[b] = second_slot;
        // Workgroup b runs on XCD b % 8 (workgroups are dealt to the eight
        // XCDs in turn), and the XCDs stream at slightly different rates:
        // per-workgroup clock reads on three boxes put XCDs 3 and 5
        // earliest, 5-8 us ahead of the latest at the end of a 523 us mean.
        // These are the three boxes' mean time per unit, XCD by XCD,
        // relative to their average.
        uint32_t xw[8] = {1029, 1023, 1027, 1015, 1028, 1019, 1028, 1023};
        if (const char *env = std::getenv("Q4RDNA_PLAN_XCD_WEIGHTS")) {  // tuning sweeps only
            uint32_t v[8];
            if (std::sscanf(env, "%u,%u,%u,%u,%u,%u,%u,%u", &v[0], &v[1], &v[2], &v[3], &v[4], &v[5], &v[6], &v[7]) ==
                8)
                std::copy(v, v + 8, xw);
        }
        for (uint32_t b = 0; b < workgroups; ++b) weight[b] = weight[b] * xw[b % 8] / 1024;
        const std::vector<uint32_t> lists = deal_items(cost, weight);
        const uint32_t head = (workgroups + 2) & ~1u;
        deal.assign(head + 2 * items, 0);
        std::copy(lists.begin(), lists.begin() + workgroups + 1, deal.begin());
        std::vector<uint32_t> owner(items);
        for (uint32_t i = 0; i < count; ++i)
            for (uint32_t item = host[i].item_begin; item < host[i + 1].item_begin; ++item) owner[item] = i;
        for (uint64_t k = 0; k < items; ++k) {
            const uint32_t item = lists[workgroups + 1 + k];
            deal[head + 2 * k] = owner[item];
            deal[head + 2 * k + 1] = item - host[owner[item]].item_begin;
        }
    }
    const uint64_t deal_off = (table_off + table_bytes + 255) & ~uint64_t(255);
    const uint64_t tail_off = (deal_off + deal.size() * sizeof(uint32_t) + 255) & ~uint64_t(255);
    std::vector<uint64_t> table(n == 1 ? groups : (groups + 1) / 2);
    for (uint32_t i = 0; i < count; ++i)
        for (uint32_t g = host[i].group_begin; g < host[i + 1].group_begin; ++g) {
            if (n == 1)
                table[g] = reinterpret_cast<uint64_t>(host[i].x + static_cast<size_t>(g - host[i].group_begin) * kGroup);
            else
                reinterpret_cast<uint32_t *>(table.data())[g] = i;
        }
    scratch += tail_off;
    DeviceGuard guard(device);
    if (!guard.ok()) return fail(Q4RDNA_ERR_HIP, "hipSetDevice(%d) failed", device);
    auto plan = std::make_unique<q4rdna_plan>();
    plan->device = device;
    plan->batch = n;
    for (uint32_t i = 0; i < count; ++i) plan->both_streams |= host[i].streams > 1 && host[i].per == 1;
    plan->count = count;
    plan->items = static_cast<uint32_t>(items);
    plan->groups = static_cast<uint32_t>(groups);
    plan->workgroups = workgroups;
    auto cleanup = [&plan]() {
        if (plan->descs) (void)hipFree(plan->descs);
        if (plan->scratch) (void)hipFree(plan->scratch);
        if (plan->sched) (void)hipFree(plan->sched);
    };
    hipError_t e = hipMalloc(&plan->descs, host.size() * sizeof(q4rdna::PlanDesc));
    if (e == hipSuccess && scratch > 0) e = hipMalloc(&plan->scratch, scratch);
    if (e == hipSuccess) e = hipMalloc(&plan->sched, 2 * sizeof(uint32_t));
    if (e != hipSuccess) {
        cleanup();
        return fail(Q4RDNA_ERR_MEMORY, "plan buffers: %s", hipGetErrorString(e));
    }
    for (uint32_t i = 0; i < count; ++i) {
        host[i].prep = plan->scratch + static_cast<uint64_t>(host[i].group_begin) * prep_per_group;
        if (host[i].per > 1) {
            host[i].partial = reinterpret_cast<float *>(plan->scratch + tail_off + part_off[i]);
            host[i].counters = reinterpret_cast<uint32_t *>(plan->scratch + tail_off + cnt_off[i]);
        }
    }
    plan->table = plan->scratch + table_off;
    plan->deal = reinterpret_cast<uint32_t *>(plan->scratch + deal_off);
    e = hipMemcpy(plan->descs, host.data(), host.size() * sizeof(q4rdna::PlanDesc), hipMemcpyHostToDevice);
    if (e == hipSuccess && scratch > 0) e = hipMemset(plan->scratch, 0, scratch);
    if (e == hipSuccess && groups > 0)
        e = hipMemcpy(plan->table, table.data(), table_bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess && !deal.empty())
        e = hipMemcpy(plan->deal, deal.data(), deal.size() * sizeof(uint32_t), hipMemcpyHostToDevice);
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
    if (plan == nullptr) return fail(Q4RDNA_ERR_ARGUMENT, "NULL plan");
    if (current_device() != plan->device)
        return fail(Q4RDNA_NOT_APPLICABLE, "plan lives on device %d, current device is %d", plan->device, current_device());
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

int q4rdna_pack(const float *w, uint32_t rows, uint32_t columns, int algorithm, uint8_t *tiles, void *stream) {
    if (w == nullptr || tiles == nullptr) return fail(Q4RDNA_ERR_ARGUMENT, "NULL input or output");
    if (!valid_shape(rows, columns)) return fail(Q4RDNA_ERR_ARGUMENT, "shape %ux%u is not 32-row x 64-column tiled", rows, columns);
    if (algorithm < Q4RDNA_ALGO_SIDECAR || algorithm > Q4RDNA_ALGO_MSE) return fail(Q4RDNA_ERR_ARGUMENT, "unknown algorithm %d", algorithm);
    if (!aligned(w, 16)) return fail(Q4RDNA_ERR_ARGUMENT, "weights must be 16-byte aligned");
    hipError_t e = q4rdna::launch_pack(w, rows, columns, algorithm, tiles, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "pack launch");
    return Q4RDNA_OK;
}

int q4rdna_dequantize(const q4rdna_weight *w, float *out, void *stream) {
    int rc = check_weight(w);
    if (rc != Q4RDNA_OK) return rc;
    if (out == nullptr || !aligned(out, 4)) return fail(Q4RDNA_ERR_ARGUMENT, "NULL or misaligned output");
    hipError_t e = q4rdna::launch_dequant(w->tiles, w->rows, w->columns, out, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "dequant launch");
    return Q4RDNA_OK;
}

}  // extern "C"
