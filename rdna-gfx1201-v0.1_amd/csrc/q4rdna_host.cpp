// Host-only logic of the Q4_RDNA runtime (see q4rdna_host.h): nothing here
// calls the HIP runtime.
#include "q4rdna_host.h"

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <queue>
#include <utility>

namespace q4rdna {
namespace host {
namespace {

int fail(std::string *error, int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    if (error) *error = buf;
    return code;
}

bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

uint64_t align256(uint64_t v) { return (v + 255) & ~uint64_t(255); }

}  // namespace

int parse_index(const uint8_t *image, uint64_t image_size, uint64_t file_size, FileHeader *header,
                std::vector<Entry> *entries, std::string *error) {
    if (image == nullptr) return fail(error, Q4RDNA_ERR_ARGUMENT, "sidecar image is NULL");
    if (image_size < sizeof(FileHeader) || file_size < sizeof(FileHeader))
        return fail(error, Q4RDNA_ERR_FORMAT, "invalid sidecar header: truncated");
    FileHeader h;
    std::memcpy(&h, image, sizeof(h));
    if (std::memcmp(h.magic, "Q4RDNA1", 8) != 0 || h.version != 1 || h.group != kGroup ||
        h.tile_rows != kTileRows || h.tile_bytes != kTileBytes)
        return fail(error, Q4RDNA_ERR_FORMAT, "invalid sidecar header");
    const uint64_t index_end = sizeof(FileHeader) + static_cast<uint64_t>(h.count) * sizeof(FileEntry);
    if (file_size < index_end) return fail(error, Q4RDNA_ERR_FORMAT, "truncated sidecar index");
    if (image_size < index_end)
        return fail(error, Q4RDNA_ERR_ARGUMENT, "image holds %llu bytes, the index ends at %llu",
                    static_cast<unsigned long long>(image_size), static_cast<unsigned long long>(index_end));
    std::vector<Entry> out;
    out.reserve(h.count);
    for (uint32_t i = 0; i < h.count; ++i) {
        FileEntry e;
        std::memcpy(&e, image + sizeof(FileHeader) + static_cast<uint64_t>(i) * sizeof(FileEntry), sizeof(e));
        // The data region's end, computed without wrapping: an entry must lie
        // inside [data_offset, data_offset + data_bytes).
        const bool inside = e.offset >= h.data_offset && e.offset - h.data_offset <= h.data_bytes &&
                            e.size <= h.data_bytes - (e.offset - h.data_offset);
        if (std::memchr(e.name, '\0', sizeof(e.name)) == nullptr || !inside || e.rows % kTileRows != 0 ||
            e.columns % kGroup != 0 || e.size != static_cast<uint64_t>(e.rows) * e.columns * 34 / kGroup)
            return fail(error, Q4RDNA_ERR_FORMAT, "invalid sidecar entry %u", i);
        out.push_back(Entry{std::string(e.name), e.rows, e.columns, e.offset, e.size});
    }
    if (h.data_offset > file_size || h.data_bytes > file_size - h.data_offset)
        return fail(error, Q4RDNA_ERR_FORMAT, "truncated sidecar data");
    if (header) *header = h;
    if (entries) *entries = std::move(out);
    return Q4RDNA_OK;
}

bool valid_shape(uint32_t rows, uint32_t cols) {
    return rows > 0 && cols > 0 && rows % kTileRows == 0 && cols % kGroup == 0;
}

uint32_t policy_split(uint32_t rows, uint32_t cols, uint32_t cus) {
    // About 32 groups per workgroup (eight waves of four tiles, all in flight
    // at once) and at most 8 chunks; more chunks only when the row tiles are
    // so few that under a quarter of the CUs would get a workgroup, fewer
    // when there would be more than six workgroups per CU.  Measured on
    // MI355X (split sweep, with and without a SwiGLU gate): 4096x4096 best at
    // 2, 1024x4096 at 2-4, 12288x4096 at 2, 4096x12288 at 6, 2048x28672 at
    // 7-8, 151936x4096 at 1-2.
    const uint32_t tiles = rows / kTileRows;
    const uint32_t groups = cols / kGroup;
    uint32_t split = std::min<uint32_t>((groups + 31) / 32, 8);
    if (static_cast<uint64_t>(tiles) * split * 4 < cus)
        split = std::min((cus / 4 + tiles - 1) / tiles, std::max<uint32_t>(1, groups / 16));
    if (static_cast<uint64_t>(tiles) * split > 6ull * cus) split = std::max<uint32_t>(1, 6 * cus / tiles);
    split = std::min(split, std::min(groups, kMaxSplit));
    return std::max<uint32_t>(split, 1);
}

std::vector<uint32_t> item_costs(const PlanLayout &layout) {
    std::vector<uint32_t> cost(layout.items);
    for (uint32_t i = 0; i < layout.count; ++i) {
        const PlanDesc &p = layout.descs[i];
        const uint32_t g = p.cols / kGroup;
        for (uint32_t item = p.item_begin; item < layout.descs[i + 1].item_begin; ++item) {
            const uint32_t part = (item - p.item_begin) % p.per;
            const uint32_t chunk = part % p.chunks;
            const uint32_t chunk_g = std::min(g, (chunk + 1) * kChunkGroups) - chunk * kChunkGroups;
            // Pairs stream four row tiles, items of both streams two per
            // stream, other items two.
            const uint32_t row_tiles = p.pair || (p.streams > 1 && p.per == 1) ? 4u : 2u;
            cost[item] = row_tiles * chunk_g + kItemEndTiles;
        }
    }
    return cost;
}

// Of the two workgroups a CU holds, the one dispatched first (b < CUs, as
// workgroups are dispatched in order) wins the CU's arbitration and streams
// faster: with equal loads on the Qwen3-8B stack, workgroups b >= CUs
// finished 20 us after the others (per-workgroup clock reads), so the CU ran
// its second workgroup alone at the end.  Workgroup b runs on XCD b % 8, and
// per-workgroup clock reads put some XCDs a few us ahead of others; the XCD
// weights are the mean relative time per unit of three boxes.
constexpr uint32_t kSecondSlotWeight = 1100;
constexpr uint32_t kXcdWeight[8] = {1029, 1023, 1027, 1015, 1028, 1019, 1028, 1023};

std::vector<uint32_t> workgroup_weights(uint32_t workgroups, uint32_t cus) {
    std::vector<uint32_t> weight(workgroups, 1024);
    for (uint32_t b = cus; b < workgroups; ++b) weight[b] = kSecondSlotWeight;
    for (uint32_t b = 0; b < workgroups; ++b) weight[b] = weight[b] * kXcdWeight[b % 8] / 1024;
    return weight;
}

// Items go in order, longest GEMV first, each to the workgroup that would
// finish it first; then moves and swaps of one item between the latest
// workgroup and an earlier one bring the latest forward while any does (each
// lowers the sorted vector of finish times, so this ends; it is capped
// besides).  On the Qwen3-8B stack (2,304 items of 192 groups x 64 rows, 9,792
// of 64 groups x 128 rows, 512 workgroups, equal weights) a round-robin deal
// leaves the most-loaded workgroup 53 units of 64 groups x 64 rows against a
// mean of 51.75; this one 52.
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

int layout_plan(const q4rdna_gemv_desc *descs, uint32_t count, uint32_t n, int device, uint32_t cus, PlanLayout *out,
                std::string *error) {
    if (out == nullptr || (descs == nullptr && count > 0))
        return fail(error, Q4RDNA_ERR_ARGUMENT, "NULL descriptors or layout");
    if (n < 1 || n > Q4RDNA_MAX_BATCH)
        return fail(error, Q4RDNA_ERR_ARGUMENT, "batch %u is outside 1..%d", n, Q4RDNA_MAX_BATCH);
    // Single vectors: 64-row blocks, kPrepBytes per group.  Batches: 256-row
    // blocks, one kBatchQuadBytesHost record per (group, quad of vectors).
    const uint32_t block_rows = n == 1 ? kBlockRows : kBatchBlockRows;
    const uint64_t prep_per_group = n == 1 ? kPrepBytes : static_cast<uint64_t>((n + 3) / 4) * kBatchQuadBytesHost;
    const uint32_t chunk_groups = n == 1 ? kChunkGroups : kBatchChunkGroups;
    for (uint32_t i = 0; i < count; ++i) {
        const q4rdna_gemv_desc &d = descs[i];
        if (d.weight.tiles == nullptr || d.x == nullptr || d.y == nullptr)
            return fail(error, Q4RDNA_ERR_ARGUMENT, "descriptor %u has a NULL pointer", i);
        if (!valid_shape(d.weight.rows, d.weight.columns) || !aligned(d.weight.tiles, 16) ||
            (d.gate_tiles != nullptr && !aligned(d.gate_tiles, 16)) || !aligned(d.x, 16) || !aligned(d.y, 4) ||
            (d.add != nullptr && !aligned(d.add, 4)))
            return fail(error, Q4RDNA_ERR_ARGUMENT, "descriptor %u: invalid shape or alignment", i);
        if (d.weight.device != device)
            return fail(error, Q4RDNA_ERR_ARGUMENT, "descriptor %u lives on device %d", i, d.weight.device);
    }
    // The GEMVs run concurrently: no y may overlap another descriptor's y,
    // x or add, and a descriptor's add is its own y or apart from it.  The
    // outputs are checked sorted by address (they must be disjoint), then
    // each input range against them by binary search.  A descriptor's x may
    // overlap its own y: the prepare launch reads every x before the sweep
    // writes any y.
    {
        struct Range {
            uintptr_t lo, hi;
            uint32_t owner;
        };
        std::vector<Range> ys(count);
        for (uint32_t i = 0; i < count; ++i) {
            const uintptr_t y0 = reinterpret_cast<uintptr_t>(descs[i].y);
            ys[i] = {y0, y0 + 4ull * n * descs[i].weight.rows, i};
        }
        std::sort(ys.begin(), ys.end(), [](const Range &a, const Range &b) { return a.lo < b.lo; });
        for (uint32_t i = 1; i < count; ++i)
            if (ys[i].lo < ys[i - 1].hi)
                return fail(error, Q4RDNA_ERR_ARGUMENT, "descriptors %u and %u: outputs overlap", ys[i - 1].owner,
                            ys[i].owner);
        // Every output that [lo, hi) meets, owner by owner.
        auto meets = [&](uintptr_t lo, uintptr_t hi, uint32_t self, bool is_add, const float *own_y) -> int {
            auto it = std::upper_bound(ys.begin(), ys.end(), lo, [](uintptr_t v, const Range &r) { return v < r.hi; });
            for (; it != ys.end() && it->lo < hi; ++it) {
                if (it->owner != self)
                    return fail(error, Q4RDNA_ERR_ARGUMENT, "descriptor %u: its %s overlaps descriptor %u's y", self,
                                is_add ? "add" : "x", it->owner);
                if (is_add && reinterpret_cast<uintptr_t>(own_y) != lo)
                    return fail(error, Q4RDNA_ERR_ARGUMENT, "descriptor %u: add overlaps y without being y", self);
            }
            return Q4RDNA_OK;
        };
        for (uint32_t i = 0; i < count; ++i) {
            const q4rdna_gemv_desc &d = descs[i];
            const uintptr_t x0 = reinterpret_cast<uintptr_t>(d.x);
            int rc = meets(x0, x0 + 4ull * n * d.weight.columns, i, false, d.y);
            if (rc == Q4RDNA_OK && d.add != nullptr) {
                const uintptr_t a0 = reinterpret_cast<uintptr_t>(d.add);
                rc = meets(a0, a0 + 4ull * n * d.weight.rows, i, true, d.y);
            }
            if (rc != Q4RDNA_OK) return rc;
        }
    }
    PlanLayout L;
    L.count = count;
    L.batch = n;
    // The GEMVs of a plan are independent, so the sweep may take them in any
    // order: GEMVs with longer items (wider K chunks) go first, so that the
    // end of the sweep, where workgroups run out of items, deals short ones.
    L.order.resize(count);
    for (uint32_t i = 0; i < count; ++i) L.order[i] = i;
    // A SwiGLU GEMV whose rows fit one chunk runs both weight streams in one
    // item per block (no split-K partials), single vectors and batches alike.
    auto both_streams = [&](uint32_t i) {
        return descs[i].gate_tiles != nullptr && descs[i].weight.columns / kGroup <= chunk_groups;
    };
    // A single-vector GEMV with no gate whose rows fit one 64-group step
    // block runs two 64-row blocks per item: half the item ends.
    auto pairs = [&](uint32_t i) {
        return n == 1 && descs[i].gate_tiles == nullptr && descs[i].weight.columns / kGroup <= 64;
    };
    auto item_groups = [&](uint32_t i) {
        return std::min(descs[i].weight.columns / kGroup, chunk_groups) * (both_streams(i) || pairs(i) ? 2u : 1u);
    };
    std::stable_sort(L.order.begin(), L.order.end(),
                     [&](uint32_t a, uint32_t b) { return item_groups(a) > item_groups(b); });
    L.descs.assign(static_cast<size_t>(count) + 1, PlanDesc{});
    L.prep_off.assign(count, 0);
    L.part_off.assign(count, 0);
    L.cnt_off.assign(count, 0);
    uint64_t items = 0, groups = 0, tail = 0;
    for (uint32_t i = 0; i < count; ++i) {
        const q4rdna_gemv_desc &d = descs[L.order[i]];
        const uint32_t g = d.weight.columns / kGroup;
        const uint32_t chunks = (g + chunk_groups - 1) / chunk_groups;
        const bool pair = pairs(L.order[i]);
        const uint32_t item_rows = pair ? 2 * block_rows : block_rows;
        const uint32_t blocks = (d.weight.rows + item_rows - 1) / item_rows;
        const uint32_t streams = d.gate_tiles != nullptr ? 2u : 1u;
        PlanDesc &p = L.descs[i];
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
        p.per = both_streams(L.order[i]) || pair ? 1u : chunks * streams;
        p.pair = pair ? 1u : 0u;
        L.prep_off[i] = groups * prep_per_group;
        if (p.per > 1) {
            L.part_off[i] = tail;
            tail = align256(tail + static_cast<uint64_t>(chunks) * streams * n * d.weight.rows * sizeof(float));
            L.cnt_off[i] = tail;
            tail += static_cast<uint64_t>(blocks) * sizeof(uint32_t);
        }
        tail = align256(tail);
        items += static_cast<uint64_t>(blocks) * p.per;
        groups += g;
        if (items > 0xffffffffull || groups * n > 0xffffffffull)
            return fail(error, Q4RDNA_ERR_ARGUMENT, "plan too large");
        L.both_streams |= p.streams > 1 && p.per == 1;
    }
    L.descs[count].item_begin = static_cast<uint32_t>(items);
    L.descs[count].group_begin = static_cast<uint32_t>(groups);
    L.items = static_cast<uint32_t>(items);
    L.groups = static_cast<uint32_t>(groups);
    // Group table of the prep launch: single vectors get each group's
    // activation address (one load, no descriptor lookup); batches the
    // descriptor index of each group.
    L.table_off = align256(groups * prep_per_group);
    L.table_bytes = groups * (n == 1 ? sizeof(uint64_t) : sizeof(uint32_t));
    L.workgroups = static_cast<uint32_t>(
        std::max<uint64_t>(1, std::min<uint64_t>(uint64_t(cus) * kPlanWorkgroupsPerCu, items)));
    // Single vectors: the items' deal to the workgroups, after the table, in
    // the kernel's form: the offsets (padded to an even count), then per item
    // its descriptor index and its index within the descriptor.
    if (n == 1) {
        const std::vector<uint32_t> lists = deal_items(item_costs(L), workgroup_weights(L.workgroups, cus));
        const uint32_t head = (L.workgroups + 2) & ~1u;
        L.deal.assign(head + 2 * items, 0);
        std::copy(lists.begin(), lists.begin() + L.workgroups + 1, L.deal.begin());
        std::vector<uint32_t> owner(items);
        for (uint32_t i = 0; i < count; ++i)
            for (uint32_t item = L.descs[i].item_begin; item < L.descs[i + 1].item_begin; ++item) owner[item] = i;
        for (uint64_t k = 0; k < items; ++k) {
            const uint32_t item = lists[L.workgroups + 1 + k];
            L.deal[head + 2 * k] = owner[item];
            L.deal[head + 2 * k + 1] = item - L.descs[owner[item]].item_begin;
        }
    }
    L.deal_off = align256(L.table_off + L.table_bytes);
    L.tail_off = align256(L.deal_off + L.deal.size() * sizeof(uint32_t));
    L.scratch_bytes = L.tail_off + tail;
    L.table.assign(n == 1 ? groups : (groups + 1) / 2, 0);
    for (uint32_t i = 0; i < count; ++i)
        for (uint32_t g = L.descs[i].group_begin; g < L.descs[i + 1].group_begin; ++g) {
            if (n == 1)
                L.table[g] = reinterpret_cast<uint64_t>(L.descs[i].x + static_cast<size_t>(g - L.descs[i].group_begin) * kGroup);
            else
                reinterpret_cast<uint32_t *>(L.table.data())[g] = i;
        }
    *out = std::move(L);
    return Q4RDNA_OK;
}

}  // namespace host
}  // namespace q4rdna
