// Host-side checks of the runtime's pure host logic (csrc/q4rdna_host.cpp),
// built with AddressSanitizer and UndefinedBehaviorSanitizer by the Makefile
// next to this file and run by tests/test_host_check.py.  No GPU is used:
// plans are laid out for descriptor lists with made-up (aligned) device
// addresses, and sidecar indexes are parsed from files.
//
//   host_check layout            lays out the plans below, checks every
//                                invariant, prints one JSON line per plan
//   host_check inspect FILE...   parses each file as a sidecar image, prints
//                                one JSON line per file (status, count, error)
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iterator>
#include <random>
#include <string>
#include <vector>

#include "q4rdna_host.h"

using q4rdna::PlanDesc;
using q4rdna::host::PlanLayout;

namespace {

int g_failures = 0;

void expect(bool ok, const char *what, const std::string &plan) {
    if (!ok) {
        ++g_failures;
        std::printf("{\"plan\": \"%s\", \"failed\": \"%s\"}\n", plan.c_str(), what);
    }
}

struct Shape {
    uint32_t rows, cols;
    bool gate, add;
};

// Descriptors with distinct, aligned made-up addresses.
std::vector<q4rdna_gemv_desc> make_descs(const std::vector<Shape> &shapes, uint32_t n) {
    std::vector<q4rdna_gemv_desc> d(shapes.size());
    uint64_t addr = 0x100000000ull;
    auto take = [&addr](uint64_t bytes) {
        const uint64_t a = addr;
        addr += (bytes + 4095) & ~uint64_t(4095);
        return a;
    };
    for (size_t i = 0; i < shapes.size(); ++i) {
        const Shape &s = shapes[i];
        const uint64_t tiles = static_cast<uint64_t>(s.rows) * s.cols * 34 / 64;
        d[i].weight.tiles = reinterpret_cast<const uint8_t *>(take(tiles));
        d[i].weight.rows = s.rows;
        d[i].weight.columns = s.cols;
        d[i].weight.device = 0;
        d[i].weight.reserved = 0;
        d[i].gate_tiles = s.gate ? reinterpret_cast<const uint8_t *>(take(tiles)) : nullptr;
        d[i].x = reinterpret_cast<const float *>(take(4ull * s.cols * n));
        d[i].add = s.add ? reinterpret_cast<const float *>(take(4ull * s.rows * n)) : nullptr;
        d[i].y = reinterpret_cast<float *>(take(4ull * s.rows * n));
    }
    return d;
}

std::vector<Shape> qwen3_stack(bool fused) {
    std::vector<Shape> s;
    for (int layer = 0; layer < 36; ++layer) {
        s.push_back({4096, 4096, false, false});   // q
        s.push_back({1024, 4096, false, false});   // k
        s.push_back({1024, 4096, false, false});   // v
        s.push_back({4096, 4096, false, false});   // o
        if (fused) {
            s.push_back({12288, 4096, true, false});  // up with the SwiGLU gate
        } else {
            s.push_back({12288, 4096, false, false});  // gate
            s.push_back({12288, 4096, false, false});  // up
        }
        s.push_back({4096, 12288, false, false});  // down
    }
    return s;
}

// A mix with every item kind: pairs, pairs with add, one-item SwiGLU,
// split-K (rows longer than one 192-group chunk) with and without a gate,
// short tails.
std::vector<Shape> mixed_plan(uint32_t seed) {
    std::mt19937 rng(seed);
    const Shape kinds[] = {{128, 512, false, false}, {256, 4096, false, true}, {192, 4096, true, false},
                           {64, 12800, false, false}, {64, 12800, true, false}, {96, 4736, false, false},
                           {224, 28672, false, true}, {32, 64, false, false}};
    std::vector<Shape> s;
    for (int i = 0; i < 600; ++i) s.push_back(kinds[rng() % 8]);
    return s;
}

uint64_t align_check(uint64_t v) { return v & 255u; }

void check_layout(const std::string &name, const std::vector<Shape> &shapes, uint32_t n, uint32_t cus) {
    const std::vector<q4rdna_gemv_desc> descs = make_descs(shapes, n);
    PlanLayout L;
    std::string error;
    const int rc = q4rdna::host::layout_plan(descs.data(), static_cast<uint32_t>(descs.size()), n, 0, cus, &L, &error);
    expect(rc == Q4RDNA_OK, "layout status", name);
    if (rc != Q4RDNA_OK) return;
    const uint32_t count = L.count;
    expect(L.descs.size() == count + 1u, "sentinel", name);
    expect(L.workgroups >= 1 && L.workgroups <= 2 * cus, "workgroups", name);
    // The order is a permutation, longest items first.
    std::vector<int> seen_desc(count, 0);
    for (uint32_t i = 0; i < count; ++i) seen_desc[L.order[i]]++;
    for (uint32_t i = 0; i < count; ++i) expect(seen_desc[i] == 1, "order is a permutation", name);
    uint64_t items = 0, groups = 0;
    bool per_one = true;
    for (uint32_t i = 0; i < count; ++i) {
        const PlanDesc &p = L.descs[i];
        const q4rdna_gemv_desc &d = descs[L.order[i]];
        expect(p.w == d.weight.tiles && p.x == d.x && p.y == d.y && p.rows == d.weight.rows, "descriptor copy", name);
        expect(p.item_begin == items && p.group_begin == groups, "item and group numbering", name);
        expect(p.prep == nullptr && p.partial == nullptr && p.counters == nullptr, "pointers unbased", name);
        expect(L.prep_off[i] == groups * (n == 1 ? q4rdna::kPrepBytes : (n + 3) / 4 * q4rdna::kBatchQuadBytesHost),
               "prep offset", name);
        items = L.descs[i + 1].item_begin;
        groups += p.cols / 64;
        per_one &= p.per == 1;
        if (p.per > 1) {
            expect(align_check(L.part_off[i]) == 0 && align_check(L.cnt_off[i]) == 0, "tail alignment", name);
            const uint64_t part_end = L.part_off[i] + 4ull * p.chunks * p.streams * n * p.rows;
            expect(part_end <= L.cnt_off[i], "partials before counters", name);
            // one counter per block: 64-row blocks for single vectors, 256-row
            // blocks for batches
            const uint64_t block_rows = n == 1 ? q4rdna::kBlockRows : q4rdna::kBatchBlockRows;
            expect(L.tail_off + L.cnt_off[i] + 4ull * ((p.rows + block_rows - 1) / block_rows) <= L.scratch_bytes,
                   "counters in scratch", name);
        }
    }
    expect(items == L.items && groups == L.groups, "totals", name);
    expect(align_check(L.table_off) == 0 && align_check(L.deal_off) == 0 && align_check(L.tail_off) == 0,
           "region alignment", name);
    expect(L.groups * (n == 1 ? q4rdna::kPrepBytes : (n + 3) / 4 * q4rdna::kBatchQuadBytesHost) <= L.table_off,
           "digits before table", name);
    expect(L.table_off + L.table_bytes <= L.deal_off, "table before deal", name);
    expect(L.deal_off + 4ull * L.deal.size() <= L.tail_off, "deal before tail", name);
    // Group table.
    for (uint32_t i = 0; i < count; ++i)
        for (uint32_t g = L.descs[i].group_begin; g < L.descs[i + 1].group_begin; ++g) {
            if (n == 1)
                expect(L.table[g] == reinterpret_cast<uint64_t>(L.descs[i].x) + 256ull * (g - L.descs[i].group_begin),
                       "group table address", name);
            else
                expect(reinterpret_cast<const uint32_t *>(L.table.data())[g] == i, "group table owner", name);
        }
    double max_load = 0.0, mean_load = 0.0;
    if (n == 1) {
        // The deal: offsets, then (descriptor, item within it) pairs; every
        // item exactly once, each workgroup's list ascending.
        const uint32_t W = L.workgroups, head = (W + 2) & ~1u;
        expect(L.deal.size() == head + 2ull * L.items, "deal size", name);
        expect(L.deal[0] == 0 && L.deal[W] == L.items, "deal ends", name);
        std::vector<int> dealt(L.items, 0);
        const std::vector<uint32_t> cost = q4rdna::host::item_costs(L);
        for (uint32_t b = 0; b < W; ++b) {
            expect(L.deal[b] <= L.deal[b + 1], "offsets ascend", name);
            uint64_t load = 0;
            int64_t prev = -1;
            for (uint32_t k = L.deal[b]; k < L.deal[b + 1] && k < L.items; ++k) {
                const uint32_t d = L.deal[head + 2 * k], local = L.deal[head + 2 * k + 1];
                expect(d < count, "entry descriptor", name);
                if (d >= count) continue;
                const uint32_t item = L.descs[d].item_begin + local;
                expect(item < L.descs[d + 1].item_begin, "entry item", name);
                if (item >= L.items) continue;
                dealt[item]++;
                expect(static_cast<int64_t>(item) > prev, "list ascends", name);
                prev = item;
                load += cost[item];
            }
            max_load = std::max<double>(max_load, static_cast<double>(load));
            mean_load += static_cast<double>(load) / W;
        }
        for (uint32_t i = 0; i < L.items; ++i) expect(dealt[i] == 1, "every item dealt once", name);
    } else {
        expect(L.deal.empty(), "batched plans have no deal", name);
    }
    std::printf("{\"plan\": \"%s\", \"gemvs\": %u, \"batch\": %u, \"items\": %u, \"groups\": %u, \"workgroups\": %u, "
                "\"scratch_bytes\": %llu, \"all_per_one\": %s, \"both_streams\": %s, \"max_load\": %.0f, "
                "\"mean_load\": %.2f}\n",
                name.c_str(), count, n, L.items, L.groups, L.workgroups,
                static_cast<unsigned long long>(L.scratch_bytes), per_one ? "true" : "false",
                L.both_streams ? "true" : "false", max_load, mean_load);
}

int run_layout() {
    check_layout("qwen3_252", qwen3_stack(false), 1, 256);
    check_layout("qwen3_216_swiglu", qwen3_stack(true), 1, 256);
    check_layout("qwen3_252_batch4", qwen3_stack(false), 4, 256);
    check_layout("qwen3_252_batch8", qwen3_stack(false), 8, 256);
    check_layout("qwen3_216_swiglu_batch8", qwen3_stack(true), 8, 256);
    check_layout("mixed", mixed_plan(7), 1, 256);
    check_layout("mixed_batch3", mixed_plan(8), 3, 256);
    check_layout("mixed_small_gpu", mixed_plan(9), 1, 8);
    check_layout("one_gemv", {{32, 64, false, false}}, 1, 256);
    // Argument errors leave the layout untouched and return a status.
    PlanLayout L;
    std::string error;
    std::vector<q4rdna_gemv_desc> bad = make_descs({{48, 64, false, false}}, 1);
    expect(q4rdna::host::layout_plan(bad.data(), 1, 1, 0, 256, &L, &error) == Q4RDNA_ERR_ARGUMENT, "bad shape", "errors");
    bad = make_descs({{32, 64, false, false}}, 1);
    bad[0].x = reinterpret_cast<const float *>(reinterpret_cast<uintptr_t>(bad[0].x) + 4);
    expect(q4rdna::host::layout_plan(bad.data(), 1, 1, 0, 256, &L, &error) == Q4RDNA_ERR_ARGUMENT, "misaligned x", "errors");
    expect(q4rdna::host::layout_plan(bad.data(), 1, 9, 0, 256, &L, &error) == Q4RDNA_ERR_ARGUMENT, "batch 9", "errors");
    bad = make_descs({{32, 64, false, false}}, 1);
    bad[0].weight.device = 1;
    expect(q4rdna::host::layout_plan(bad.data(), 1, 1, 0, 256, &L, &error) == Q4RDNA_ERR_ARGUMENT, "other device", "errors");
    // Aliasing: outputs overlapping each other, another descriptor's x or
    // add on a y, an add that overlaps its own y without being it.  Shared
    // x, a descriptor's x on its own y and an add that is its own y are fine.
    const std::vector<Shape> two = {{64, 512, false, true}, {64, 512, false, true}};
    std::vector<q4rdna_gemv_desc> d2 = make_descs(two, 2);
    expect(q4rdna::host::layout_plan(d2.data(), 2, 2, 0, 256, &L, &error) == Q4RDNA_OK, "disjoint", "aliasing");
    bad = d2;
    bad[1].y = bad[0].y + 32;
    expect(q4rdna::host::layout_plan(bad.data(), 2, 2, 0, 256, &L, &error) == Q4RDNA_ERR_ARGUMENT, "outputs overlap",
           "aliasing");
    bad = d2;
    bad[1].x = reinterpret_cast<const float *>(bad[0].y);
    expect(q4rdna::host::layout_plan(bad.data(), 2, 2, 0, 256, &L, &error) == Q4RDNA_ERR_ARGUMENT,
           "x on another's y", "aliasing");
    bad = d2;
    bad[1].add = bad[0].y + 1;
    expect(q4rdna::host::layout_plan(bad.data(), 2, 2, 0, 256, &L, &error) == Q4RDNA_ERR_ARGUMENT,
           "add on another's y", "aliasing");
    bad = d2;
    bad[0].add = bad[0].y + 4;
    expect(q4rdna::host::layout_plan(bad.data(), 2, 2, 0, 256, &L, &error) == Q4RDNA_ERR_ARGUMENT,
           "add shifted on its own y", "aliasing");
    std::vector<q4rdna_gemv_desc> ok = d2;
    ok[1].x = ok[0].x;    // a shared activation
    ok[0].add = ok[0].y;  // the residual in place
    expect(q4rdna::host::layout_plan(ok.data(), 2, 2, 0, 256, &L, &error) == Q4RDNA_OK, "shared x, add is y",
           "aliasing");
    ok = d2;
    ok[0].x = reinterpret_cast<const float *>(ok[0].y);  // read by the prepare launch before the sweep writes y
    expect(q4rdna::host::layout_plan(ok.data(), 2, 2, 0, 256, &L, &error) == Q4RDNA_OK, "x on its own y",
           "aliasing");
    std::printf("{\"failures\": %d}\n", g_failures);
    return g_failures == 0 ? 0 : 1;
}

int run_inspect(int argc, char **argv) {
    for (int i = 0; i < argc; ++i) {
        std::ifstream in(argv[i], std::ios::binary);
        std::vector<uint8_t> image((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
        q4rdna::host::FileHeader h{};
        std::vector<q4rdna::host::Entry> entries;
        std::string error;
        // Copy into an exactly sized heap block so reads past the image end
        // are caught by the sanitizer.
        uint8_t *exact = static_cast<uint8_t *>(std::malloc(image.size() ? image.size() : 1));
        if (!image.empty()) std::memcpy(exact, image.data(), image.size());
        const int rc = q4rdna::host::parse_index(exact, image.size(), image.size(), &h, &entries, &error);
        std::free(exact);
        std::printf("{\"file\": \"%s\", \"status\": %d, \"count\": %u, \"error\": \"%s\"}\n", argv[i], rc,
                    rc == Q4RDNA_OK ? static_cast<unsigned>(entries.size()) : 0u, error.c_str());
    }
    return 0;
}


// The exchange tree's protocol, run on the CPU with the kernels' own shape
// functions (exchange_leaves, exchange_meets): for every split 2..64 and
// random interleavings of the chunks' exchanges, one chunk clears the root,
// every slot region used is swapped into exactly twice (so all are empty
// again), split - 1 regions take part, all indices lie inside
// exchange_nodes(split) regions, and the root's sum -- kept as the
// expression it adds up, each node writing its two operands in a fixed
// order since fp32 addition is commutative -- is the same in every
// interleaving.
// `meets` is the shape rule under test: the kernels' exchange_meets, or a
// planted mistake that the check must catch.
using MeetsFn = bool (*)(uint32_t, uint32_t, uint32_t, uint32_t);
bool planted_off_by_one(uint32_t node, uint32_t d, uint32_t leaves, uint32_t split) {
    return (node & 1u) != 0u || ((node + 1u) << d) - leaves <= split;
}
bool planted_always(uint32_t, uint32_t, uint32_t, uint32_t) { return true; }
bool real_meets(uint32_t node, uint32_t d, uint32_t leaves, uint32_t split) {
    return q4rdna::exchange_meets(node, d, leaves, split);
}

int run_tree(MeetsFn meets) {
    std::mt19937 rng(12345);
    int splits = 0;
    for (uint32_t split = 2; split <= q4rdna::host::kMaxSplit; ++split) {
        const uint32_t P = q4rdna::exchange_leaves(split);
        std::string first;
        bool ok = true;
        for (int trial = 0; trial < 200 && ok; ++trial) {
            std::vector<std::string> slot(P - 1), val(split);
            std::vector<int> swaps(P - 1, 0);
            std::vector<uint32_t> node(split), depth(split, 0);
            std::vector<uint32_t> alive;
            for (uint32_t s = 0; s < split; ++s) {
                val[s] = "p" + std::to_string(s);
                node[s] = P + s;
                alive.push_back(s);
            }
            std::vector<std::string> roots;
            while (!alive.empty()) {
                const size_t pick = rng() % alive.size();
                const uint32_t s = alive[pick];
                // Advance chunk s to its next meeting (or past the root).
                while (node[s] > 1u && !meets(node[s], depth[s], P, split)) {
                    node[s] >>= 1;
                    ++depth[s];
                }
                if (node[s] <= 1u) {
                    roots.push_back(val[s]);
                    alive.erase(alive.begin() + pick);
                    continue;
                }
                const uint32_t region = (node[s] >> 1) - 1u;
                ok = ok && region < q4rdna::host::exchange_nodes(split);
                if (!ok) break;
                ++swaps[region];
                node[s] >>= 1;
                ++depth[s];
                if (slot[region].empty()) {
                    slot[region] = val[s];
                    alive.erase(alive.begin() + pick);
                } else {
                    const std::string &a = slot[region], &b = val[s];
                    val[s] = a < b ? "(" + a + "+" + b + ")" : "(" + b + "+" + a + ")";
                    slot[region].clear();
                }
            }
            int used = 0;
            for (size_t k = 0; k < slot.size(); ++k) {
                ok = ok && slot[k].empty() && (swaps[k] == 0 || swaps[k] == 2);
                used += swaps[k] == 2;
            }
            ok = ok && roots.size() == 1 && used == static_cast<int>(split) - 1;
            if (ok && trial == 0) first = roots[0];
            ok = ok && roots[0] == first;
        }
        expect(ok, "tree protocol", ("split " + std::to_string(split)).c_str());
        if (split == 6) std::printf("{\"split\": 6, \"root\": \"%s\"}\n", first.c_str());
        ++splits;
    }
    std::printf("{\"tree_splits\": %d, \"failures\": %d}\n", splits, g_failures);
    return g_failures == 0 ? 0 : 1;
}

}  // namespace

int main(int argc, char **argv) {
    if (argc >= 2 && std::strcmp(argv[1], "layout") == 0) return run_layout();
    if (argc >= 2 && std::strcmp(argv[1], "inspect") == 0) return run_inspect(argc - 2, argv + 2);
    if (argc >= 2 && std::strcmp(argv[1], "tree") == 0) return run_tree(real_meets);
    // Planted mistakes in the shape rule: each must be reported as failures.
    if (argc >= 2 && std::strcmp(argv[1], "tree-planted-off-by-one") == 0) return run_tree(planted_off_by_one);
    if (argc >= 2 && std::strcmp(argv[1], "tree-planted-always") == 0) return run_tree(planted_always);
    std::fprintf(stderr, "usage: host_check layout | inspect FILE... | tree | tree-planted-off-by-one | "
                         "tree-planted-always\n");
    return 2;
}
