// Internal interface between the host runtime (q4rdna_runtime.cpp) and the
// gfx950 kernels (q4rdna_kernels.hip).  Not part of the C ABI.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

namespace q4rdna {

constexpr uint32_t kGroup = 64;
constexpr uint32_t kTileRows = 32;
constexpr uint32_t kTileBytes = 1088;

// Exchange slots of two-chunk split-K launches: a partial sum p is stored as
// bits(p) XOR kSlotKey, so every word is zero between launches and memory
// that was zero-filled (a memset, a zero-initialised device array) is a valid
// set of empty slots.  kSlotKey is a signaling-NaN pattern, which arithmetic
// never produces; a partial with exactly those bits would store as zero, so
// it is sent as kSlotQuietNan instead.
constexpr uint32_t kSlotKey = 0x7fa5a5a5u;
constexpr uint32_t kSlotQuietNan = 0x7fc00000u;

// The exchange tree's shape, shared by the kernels (exchange_tree) and the
// host (slot sizing, the sanitizer check's simulation).  The `split` >= 2
// K chunks of a row are the leaves P + s of a heap over P =
// exchange_leaves(split) leaves; internal node k (1 <= k < P) owns slot
// region k - 1.  Going up from a leaf, node `node` at depth d (0 = the
// leaves) meets its sibling's subtree in its parent's slot unless it is a
// left child whose right sibling's first leaf, (node + 1) << d, lies past
// the last chunk; then the value passes straight up.
__host__ __device__ constexpr uint32_t exchange_leaves(uint32_t split) {
    uint32_t p = 1;
    while (p < split) p <<= 1;
    return p;
}
__host__ __device__ constexpr bool exchange_meets(uint32_t node, uint32_t d, uint32_t leaves, uint32_t split) {
    return (node & 1u) != 0u || ((node + 1u) << d) - leaves < split;
}

// One GEMV launch.  gate != nullptr selects SwiGLU, add != nullptr the bias
// epilogue.  split > 1 K chunks meet in an exchange tree over
// slots[exchange_nodes(split) * vectors * rows (x2 with gate)] (vectors is 1
// outside gemv_multi_kernel), zero on entry and left zero.
struct GemvArgs {
    const uint8_t *w;
    const uint8_t *gate;
    const float *x;
    const float *add;
    float *y;
    uint32_t rows;
    uint32_t cols;
    uint32_t split;
    uint32_t *slots;
    uint32_t short_waves;  // waves per workgroup: 8 or 4 for K chunks of at most 64 groups,
                           // 16 for chunks of 65..128 groups (gemv_waves)
    uint32_t vectors;      // launch_gemv_multi: activation vectors (x [vectors][cols], y/add [vectors][rows])
    uint32_t split_magic;  // split_magic(split)
    uint32_t clock_slot;   // the clock build's record slot for this launch
};

// Device-side descriptor of one GEMV in a multi-tensor plan.  Work items are
// (64-row block, stream, K chunk of up to kChunkGroups groups), numbered from
// item_begin block-major, then stream (0 = w, 1 = the SwiGLU gate), then
// chunk; `per` items per block.  A single-vector SwiGLU GEMV whose rows fit
// one chunk has per = 1: its item streams both weights.  A `pair` GEMV
// (single vector, no gate, rows of at most 64 groups) has items of two
// 64-row blocks, numbered from item_begin, one per 128 rows.  The activation is
// first converted into int8 digits (kPrepBytes per 64-element group) in
// `prep`.  When a block has more than one item (per > 1) its items meet in
// partial[stream][chunk][rows] through counters[block], zero between
// launches.
struct PlanDesc {
    const uint8_t *w;
    const uint8_t *gate;
    const float *x;
    const float *add;
    float *y;
    uint8_t *prep;
    float *partial;
    uint32_t *counters;
    uint32_t rows;
    uint32_t cols;
    uint32_t item_begin;
    uint32_t group_begin;
    uint32_t chunks;
    uint32_t streams;
    uint32_t per;
    uint32_t pair;  // single vector, no gate, one chunk: an item covers two 64-row blocks (128 rows)
};

// The single-vector sweep's arithmetic: the int8-MFMA formulation, or, in
// the library built with -DQ4RDNA_SWEEP_VALU (make valu-sweep; kept for
// the MFMA-against-VALU measurement of the sweep), the per-tensor kernels'
// VALU formulation on fp32 activations laid out by the prepare launch.
#if defined(Q4RDNA_SWEEP_VALU)
constexpr bool kSweepValu = true;
constexpr uint32_t kPrepBytes = 288;  // VALU layout: 16 float4 of scaled x + 8 lane sums
#else
constexpr bool kSweepValu = false;
constexpr uint32_t kPrepBytes = 272;  // int8 digits (256) + the group factor (16)
#endif
// The library built with -DQ4RDNA_SWEEP_CLOCKS (make sweep-clocks, "the
// clock build") records each single-vector sweep workgroup's first and last
// clock (s_memrealtime, 100 MHz) of the latest launch, for up to
// kMaxSweepClocks workgroups, and for the single-launch kernels (gemv_kernel's
// short-range path, gemv_group_kernel) each workgroup's clocks at its start,
// once x is staged, once its rows are reduced and at its end, with its
// HW_ID, in launch slot clock_slot (one of kGemvClockSlots, given per launch
// by the host); the product build records nothing.
#if defined(Q4RDNA_SWEEP_CLOCKS)
constexpr bool kSweepClocks = true;
#else
constexpr bool kSweepClocks = false;
#endif
constexpr uint32_t kMaxSweepClocks = 4096;
constexpr uint32_t kGemvClockSlots = 256;
constexpr uint32_t kGemvClockWorkgroups = 1024;
constexpr uint32_t kGemvClockWords = 6;  // start, staged, reduced, end, HW_ID, grid size
// K chunk of a single-vector plan item: 192 groups holds a whole 12288-wide
// row in one item, so such GEMVs need no split-K partials.
constexpr uint32_t kChunkGroups = 192;
constexpr uint32_t kBlockRows = 64;

// The kernels divide by the split with a multiply: magic = ceil(2^32 /
// split) (0 for split 1) gives n / split exactly for n * split < 2^32, which
// gemv_shape_fits guarantees for every n they divide (the workgroup index
// and s * groups).
inline uint32_t split_magic(uint32_t split) {
    return split <= 1 ? 0u : static_cast<uint32_t>(((uint64_t{1} << 32) + split - 1) / split);
}
inline bool gemv_shape_fits(uint64_t row_tiles, uint64_t groups, uint64_t split) {
    return row_tiles * split * split < (uint64_t{1} << 32) && groups * split * split < (uint64_t{1} << 32);
}
hipError_t launch_gemv(const GemvArgs &args, hipStream_t stream);
// The reference's old mapping, one thread per row in k order (split 1; the
// split-K fields are unused).
hipError_t launch_gemv_sequential(const GemvArgs &args, hipStream_t stream);
// GemvArgs::short_waves for rows of `groups` groups split into `split` K
// chunks, `workgroups` in all on `cus` CUs.
uint32_t gemv_waves(uint32_t groups, uint32_t split, uint64_t workgroups, uint32_t cus);
// args.vectors = 2..8 activation vectors; every K chunk (args.split of them)
// must hold at most gemv_multi_stage_groups(args.vectors) groups.
hipError_t launch_gemv_multi(const GemvArgs &args, hipStream_t stream);
uint32_t gemv_multi_stage_groups(uint32_t vectors);
// descs[count] plus a sentinel whose item_begin / group_begin are the totals.
// The prep launch converts every activation into digits: group g of the
// plan (global numbering) reads its 64 floats at group_x[g] and writes
// kPrepBytes at prep + g * kPrepBytes.  The plan launch then sweeps the
// items, dealt to its workgroups by the plan: deal holds workgroups + 1
// offsets (padded to an even count), then one (descriptor index, item within
// the descriptor) pair of uint32 per item; workgroup b runs entries
// [deal[b], deal[b + 1]), in increasing item order.  The batched sweep takes items from a queue instead: sched
// holds its two zeroed counters, owned by the plan (left zero after every
// launch).
hipError_t launch_prep(const float *const *group_x, uint8_t *prep, uint32_t groups, hipStream_t stream);
// both_streams: some GEMV has per == 1 with a SwiGLU gate (one item streams
// both weights); plans without such GEMVs run a sweep built without that path.
hipError_t launch_plan(const PlanDesc *descs, const uint32_t *deal, uint32_t workgroups, bool both_streams,
                       hipStream_t stream);
// Cost of one single-vector item in the deal: 1,088-byte tiles it streams
// plus a fixed charge for its end (reduction, stores, barrier), measured at
// about the time one workgroup takes to stream eight tiles.
constexpr uint32_t kItemEndTiles = 8;
// Batched plans (n = 2..8 activation vectors per GEMV; x [n][cols],
// y and add [n][rows]): items are 256-row blocks, prep holds
// kBatchQuadBytesHost per (group, quad of 4 vectors).
constexpr uint32_t kBatchQuadBytesHost = 1040;
constexpr uint32_t kBatchBlockRows = 256;
constexpr uint32_t kBatchChunkGroups = 192;  // K chunk of a batched item (a whole 12288-wide row)
hipError_t launch_prep_batch(const PlanDesc *descs, const uint32_t *owner, uint32_t groups, uint32_t n,
                             hipStream_t stream);
hipError_t launch_plan_batch(const PlanDesc *descs, uint32_t items, uint32_t n, uint32_t workgroups, uint32_t *sched,
                             hipStream_t stream);
constexpr uint32_t kMaxGroup = 8;  // GEMVs of one group launch (Q4RDNA_MAX_GROUP)

// A VALU group launch (gemv_kernel's arithmetic): up to kMaxGroup GEMVs
// sharing x of `cols` floats, the row tiles of all of them numbered GEMV by
// GEMV from tile_begin (`tiles` in all), each split into `split` K chunks of
// at most kGroupChunkGroups groups.  The chunks of a row tile meet as in
// gemv_kernel: in an exchange tree over slots[exchange_nodes(split) * rows
// (x2 with gate)] per GEMV.  gate is given for every GEMV or for none; add
// may be null per GEMV.
constexpr uint32_t kGroupChunkGroups = 64;
struct GemvGroupEntry {
    const uint8_t *w;
    const uint8_t *gate;
    const float *add;
    float *y;
    uint32_t *slots;
    uint32_t rows;
    uint32_t tile_begin;
};
struct GemvGroupArgs {
    GemvGroupEntry g[kMaxGroup];
    const float *x;
    uint32_t count, cols, split, tiles;
    uint32_t short_waves;  // 8 or 4, as GemvArgs::short_waves
    uint32_t split_magic;  // split_magic(split)
    uint32_t clock_slot;   // as GemvArgs::clock_slot
};
hipError_t launch_gemv_group(const GemvGroupArgs &args, hipStream_t stream);

hipError_t launch_dequant(const uint8_t *w, uint32_t rows, uint32_t cols, float *out,
                          hipStream_t stream);
hipError_t launch_pack(const float *w, uint32_t rows, uint32_t cols, int algorithm, uint8_t *tiles,
                       hipStream_t stream);

// Workgroups of 256 threads the kernels are built for, and the number the
// plan kernel launches per CU: with the fixed item deal the grid must be
// exactly two workgroups per CU (a third on some CUs runs its share slower).
constexpr uint32_t kThreads = 256;
constexpr uint32_t kPlanWorkgroupsPerCu = 2;

}  // namespace q4rdna
