// Host-only logic of the Q4_RDNA runtime: sidecar index parsing, the
// per-tensor split policy and the multi-tensor plan layout with its item
// deal.  Nothing here calls the HIP runtime, so the same code builds into the
// product library and into the sanitizer-instrumented host check
// (tests/host_check).  Not part of the C ABI.
#pragma once

#include <stdint.h>

#include <string>
#include <vector>

#include "q4rdna.h"
#include "q4rdna_internal.h"

namespace q4rdna {
namespace host {

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

// Validate a header + index held in image[0, image_size) of a file of
// file_size bytes: the loader rules of source/q4rdna.cu:129-155 and the
// data-length check of :163-170.  Returns a Q4RDNA_* status; *error
// describes a failure.
int parse_index(const uint8_t *image, uint64_t image_size, uint64_t file_size, FileHeader *header,
                std::vector<Entry> *entries, std::string *error);

bool valid_shape(uint32_t rows, uint32_t cols);

constexpr uint32_t kMaxSplit = 64;

// Exchange-slot regions of a launch whose K chunks meet in a binary tree
// (the per-tensor and group kernels): one per internal node of a heap over
// the smallest power of two >= split, so split - 1 of them take part; none
// without a split.
constexpr uint32_t exchange_nodes(uint32_t split) { return exchange_leaves(split) - 1; }

// Split-K factor of a per-tensor launch of rows x cols on a GPU with `cus`
// compute units.
uint32_t policy_split(uint32_t rows, uint32_t cols, uint32_t cus);

// Everything a plan is made of, computed on the host.  Scratch regions are
// byte offsets from the start of the plan's scratch buffer, all 256-byte
// aligned:
//   [0, table_off)                 activation digits (prep_off[i] per GEMV)
//   [table_off, +table_bytes)      the prep launch's group table
//   [deal_off, +deal.size() * 4)   single-vector plans: the item deal
//   [tail_off, scratch_bytes)      split-K partials and counters
// descs[i] describes the caller's descriptor order[i] (longest items first),
// descs[count] is the sentinel; its prep / partial / counters pointers are
// null until the runtime bases them on the allocated scratch.
struct PlanLayout {
    uint32_t count = 0, batch = 1, items = 0, groups = 0, workgroups = 0;
    bool both_streams = false;
    std::vector<uint32_t> order;
    std::vector<PlanDesc> descs;
    std::vector<uint64_t> prep_off, part_off, cnt_off;  // per plan GEMV; part/cnt only where per > 1
    std::vector<uint64_t> table;  // group table: activation address per group (single vectors) or
                                  // descriptor index per group, two uint32 per word (batches)
    uint64_t table_off = 0, table_bytes = 0, deal_off = 0, tail_off = 0, scratch_bytes = 0;
    std::vector<uint32_t> deal;  // single vectors: see launch_plan in q4rdna_internal.h
};

// Item costs of a single-vector plan (one per item, in item order).
std::vector<uint32_t> item_costs(const PlanLayout &layout);

// Time per unit of item cost of each of the plan's workgroups (1024 = 1).
std::vector<uint32_t> workgroup_weights(uint32_t workgroups, uint32_t cus);

// Deal of a single-vector sweep's items to its workgroups.  cost[i] is item
// i's weight in the sweep; weight[b] is workgroup b's time per unit of cost.
// Returns per workgroup the offset of its list (workgroups + 1 offsets) and
// the lists, each in increasing item order.
std::vector<uint32_t> deal_items(const std::vector<uint32_t> &cost, const std::vector<uint32_t> &weight);

// Lay out a plan of `count` descriptors with n activation vectors each for a
// device with `cus` compute units.  Returns a Q4RDNA_* status.
int layout_plan(const q4rdna_gemv_desc *descs, uint32_t count, uint32_t n, int device, uint32_t cus, PlanLayout *out,
                std::string *error);

}  // namespace host
}  // namespace q4rdna
