// gfx950 (CDNA4) kernels for the Q4_RDNA group-64 dequant-GEMV.
//
// Tile layout (restated from source/q4rdna.cu:20-24,346,359,370): row tile rt
// and group g form tile t = rt*G + g of 1088 bytes: 32 fp16 scales (row lane
// l at byte 2l), then byte 64 + 32*i + l holds the codes of k = 64g + 2i (low
// nibble) and 2i+1 (high nibble), two's complement in [-8, 7].
//
// Wave64 mapping.  One wave consumes one whole tile per step.  Lane
// (q = lane & 7, a = lane >> 3) loads four dwords at 64 + 32*(a + 8j) + 4q,
// j = 0..3: rows 4q..4q+3 at k-pairs i = a, a+8, a+16, a+24.  For each j one
// load instruction reads one contiguous 256-byte block of the tile, so the
// 1024 code bytes arrive in four fully coalesced loads, plus one 8-byte load
// of the lane's four scales.
//
// Decode.  XOR 0x88888888 turns every nibble into offset binary u = q + 8.
// Masked in place, a nibble in bits 0-3 (4-7) of a 16-bit half is the fp16
// subnormal u * 2^-24 (16u * 2^-24), exact; rows 4q and 4q+2 sit in the
// halves of the dword itself, rows 4q+1 and 4q+3 in the halves of the dword
// shifted right by 8.  So a dword of 8 codes becomes four f16x2 registers
// with one shift and four masks, and each weight takes one v_fma_mix_f32
// (fp16 operand, fp32 product and sum).  The 2^24 and the 1/16 of the high
// nibbles are folded into the staged activation (x * 2^24 for even k,
// x * 2^20 for odd k): every product is exactly u * x, so every partial sum
// is the one of a float(u) * x loop.  The -8 offset is folded into a
// per-(group, lane) constant c = -8 * sum of the lane's eight x values, and
// the fp16 scale multiplies the lane's per-(row, group) partial once per
// group.  The staged activation is finite for |x| < 2^104.
//
// Activations.  The workgroup stages x for up to 64 groups at a time in LDS,
// rearranged so lane a reads its 4 even-k values, its 4 odd-k values (/16)
// and c with two ds_read_b128 and one ds_read_b32 (8 lanes share each
// address, a broadcast).
//
// Workgroups.  A K chunk of at most 64 groups is taken by eight waves (four
// when the launch has many workgroups per CU) with every load issued before
// the first wait; longer chunks by four waves that keep two tile batches in
// flight.
//
// Reduction.  Lane partials are summed over a with xor-8/16/32 cross-lane
// adds (a DPP row rotate and two permlane swaps), the waves' results in LDS
// in wave order, and K chunks split across workgroups meet in a fixed binary
// tree of atomic exchange slots (exchange_tree), so every result is
// bit-reproducible run to run.
#include <type_traits>

#include "q4rdna_device.h"

namespace q4rdna {
namespace {

constexpr int kWaves = 4;       // waves of the pipelined loop's workgroup
constexpr int kShortWaves = 8;  // waves of the short-range kernel's workgroup
constexpr int kWideWaves = 16;  // waves of the wide short-range workgroup (one per CU, chunks up to 128 groups)
constexpr int kStageGroups = 64;  // groups of x staged in LDS at once
constexpr int kWideStageGroups = 128;
constexpr int kBatch = 2;         // default tiles per wave per loop trip (x2 in flight)

template <int SG>
struct XStageT {
    float4 v[SG][16];  // [g][a] even-k x * 2^24, [g][8 + a] odd-k x * 2^20
    float c[SG][8];    // -8 * sum of the lane's 8 x values
};
using XStage = XStageT<kStageGroups>;

struct TileRegs {
    uint32_t d[4];
    uint32_t s01, s23;
};

// The clock build's phase clocks of a single-launch workgroup (see
// kGemvClockSlots): read at its start, once x is staged, once its rows are
// reduced, and at its end; the product build compiles them away.
struct PhaseClocks {
    uint64_t t[4];
};
__device__ __forceinline__ void phase_clock(PhaseClocks &c, int i) {
    if constexpr (kSweepClocks) c.t[i] = __builtin_amdgcn_s_memrealtime();
}
#if defined(Q4RDNA_SWEEP_CLOCKS)
__device__ uint64_t g_gemv_clocks[kGemvClockSlots][kGemvClockWorkgroups][kGemvClockWords];
#endif
// After every thread has finished: the end clock, then thread 0 stores the
// workgroup's record with one vector store per word.
__device__ __forceinline__ void phase_record(PhaseClocks &c, uint32_t slot) {
#if defined(Q4RDNA_SWEEP_CLOCKS)
    __syncthreads();
    phase_clock(c, 3);
    if (threadIdx.x == 0 && blockIdx.x < kGemvClockWorkgroups && slot < kGemvClockSlots) {
        uint64_t *r = g_gemv_clocks[slot][blockIdx.x];
        for (int i = 0; i < 4; ++i) r[i] = c.t[i];
        r[4] = __builtin_amdgcn_s_getreg((31 << 11) | 4);  // HW_REG_HW_ID, all 32 bits
        r[5] = gridDim.x;
    }
#else
    (void)c;
    (void)slot;
#endif
}

// Weights are read exactly once per GEMV: nontemporal loads stream them past
// the caches instead of evicting the activations and partial sums.
__device__ __forceinline__ TileRegs load_tile(const uint8_t *__restrict__ tile, int q, int a) {
    TileRegs r;
    // One 32-bit lane offset on the (wave-uniform) tile address.
    const uint32_t lane_off = 64u + 4u * static_cast<uint32_t>(q) + 32u * static_cast<uint32_t>(a);
#pragma unroll
    for (int j = 0; j < 4; ++j) r.d[j] = __builtin_nontemporal_load((gptr_u32)(tile + (lane_off + 256u * j)));
    const u32x2 s = __builtin_nontemporal_load((gptr_u32x2)(tile + 8u * static_cast<uint32_t>(q)));
    r.s01 = s.x;
    r.s23 = s.y;
    return r;
}

__device__ __forceinline__ void tile_fma(const TileRegs &r, const float4 xl, const float4 xh, const float c,
                                         float (&acc)[4]) {
    apply_codes(split_codes(r.d), r.s01, r.s23, xl, xh, c, acc);
}

// Stage x for groups [g0, g0 + ng) into LDS.
__device__ __forceinline__ void stage_x(XStage &st, const float *__restrict__ x, uint32_t g0, int ng) {
    for (int idx = threadIdx.x; idx < ng * 8; idx += kThreads) {
        const int g = idx >> 3, a = idx & 7;
        const gptr_cf32 b = (gptr_cf32)x + (static_cast<size_t>(g0) + g) * kGroup + 2 * a;
        const float l0 = b[0], h0 = b[1], l1 = b[16], h1 = b[17];
        const float l2 = b[32], h2 = b[33], l3 = b[48], h3 = b[49];
        st.v[g][a] = make_float4(l0 * kEvenScale, l1 * kEvenScale, l2 * kEvenScale, l3 * kEvenScale);
        st.v[g][8 + a] = make_float4(h0 * kOddScale, h1 * kOddScale, h2 * kOddScale, h3 * kOddScale);
        st.c[g][a] = -8.0f * (((((((l0 + h0) + l1) + h1) + l2) + h2) + l3) + h3);
    }
}

template <int SG, int WR>
struct SharedT {
    XStageT<SG> st;
    float red[2][WR][32];
};
using Shared = SharedT<kStageGroups, kShortWaves>;
// The workgroup's shared memory for W waves.
template <int W>
using SharedFor = std::conditional_t<(W > kShortWaves), SharedT<kWideStageGroups, kWideWaves>, Shared>;

template <bool GATE, int BATCH>
__device__ __forceinline__ void load_batch(TileRegs (&t)[BATCH], TileRegs (&u)[BATCH],
                                           const uint8_t *__restrict__ wt, const uint8_t *__restrict__ gt,
                                           uint32_t s0, int g, int ng, int q, int a) {
#pragma unroll
    for (int b = 0; b < BATCH; ++b) {
        const int gg = g + kWaves * b;
        if (gg < ng) {
            t[b] = load_tile(wt + static_cast<size_t>(s0 + gg) * kTileBytes, q, a);
            if constexpr (GATE) u[b] = load_tile(gt + static_cast<size_t>(s0 + gg) * kTileBytes, q, a);
        }
    }
}

template <bool GATE, int BATCH>
__device__ __forceinline__ void compute_batch(const TileRegs (&t)[BATCH], const TileRegs (&u)[BATCH],
                                              const XStage &st, int g, int ng, int a, float (&acc)[4],
                                              float (&gacc)[4]) {
#pragma unroll
    for (int b = 0; b < BATCH; ++b) {
        const int gg = g + kWaves * b;
        if (gg < ng) {
            const float4 xl = st.v[gg][a];
            const float4 xh = st.v[gg][8 + a];
            const float c = st.c[gg][a];
            tile_fma(t[b], xl, xh, c, acc);
            if constexpr (GATE) tile_fma(u[b], xl, xh, c, gacc);
        }
    }
}

// Sum the lanes' row partials of a row tile over the workgroup: xor-8/16/32
// cross-lane adds within each wave, then the W waves in wave order through LDS.
// Threads 0..31 return the row sums (out, gout).
template <bool GATE, int W, class Sh>
__device__ __forceinline__ void reduce_rows(Sh &sh, float (&acc)[4], float (&gacc)[4], float &out, float &gout) {
    const int lane = threadIdx.x & 63, wave = wave_id();
    // Lane l ends with row 4 (l & 7) + (l >> 4); lanes l and l ^ 8 agree.
    const float tot = add_over_a4(acc);
    float gtot = 0.f;
    if constexpr (GATE) gtot = add_over_a4(gacc);
    if ((lane & 8) == 0) {
        const int row = 4 * (lane & 7) + (lane >> 4);
        sh.red[0][wave][row] = tot;
        if constexpr (GATE) sh.red[1][wave][row] = gtot;
    }
    __syncthreads();
    if (threadIdx.x < 32) {
        const int t = threadIdx.x;
        float v = sh.red[0][0][t];
#pragma unroll
        for (int wv = 1; wv < W; ++wv) v += sh.red[0][wv][t];
        out = v;
        if constexpr (GATE) {
            float gv = sh.red[1][0][t];
#pragma unroll
            for (int wv = 1; wv < W; ++wv) gv += sh.red[1][wv][t];
            gout = gv;
        }
    }
}


// Partial dot products of row tile `rt` over groups [g_begin, g_end), summed
// over the workgroup.  Threads 0..31 return the row partials (out, gout).
// Wave w takes groups g_begin + w, + 4, ...; each wave keeps the next batch
// of tiles in flight while it converts the current one, and the first batch
// is issued before the activations are staged.
template <bool GATE, int BATCH = kBatch>
__device__ __forceinline__ void tile_row_partial(Shared &sh, const uint8_t *__restrict__ w,
                                                 const uint8_t *__restrict__ gw,
                                                 const float *__restrict__ x, uint32_t cols,
                                                 uint32_t rt, uint32_t g_begin, uint32_t g_end,
                                                 float &out, float &gout) {
    const uint32_t groups = cols / kGroup;
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int q = lane & 7, a = lane >> 3;
    const size_t row_tile_offset = static_cast<size_t>(rt) * groups * kTileBytes;
    const uint8_t *wt = w + row_tile_offset;
    const uint8_t *gt = GATE ? gw + row_tile_offset : nullptr;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    float gacc[4] = {0.f, 0.f, 0.f, 0.f};

    for (uint32_t s0 = g_begin; s0 < g_end; s0 += kStageGroups) {
        const int ng = static_cast<int>(min(static_cast<uint32_t>(kStageGroups), g_end - s0));
        TileRegs cur[BATCH], gcur[BATCH];
        load_batch<GATE, BATCH>(cur, gcur, wt, gt, s0, wave, ng, q, a);
        __syncthreads();
        stage_x(sh.st, x, s0, ng);
        __syncthreads();
        for (int g = wave; g < ng; g += kWaves * BATCH) {
            TileRegs nxt[BATCH], gnxt[BATCH];
            const int gn = g + kWaves * BATCH;
            if (gn < ng) load_batch<GATE, BATCH>(nxt, gnxt, wt, gt, s0, gn, ng, q, a);
            compute_batch<GATE, BATCH>(cur, gcur, sh.st, g, ng, a, acc, gacc);
#pragma unroll
            for (int b = 0; b < BATCH; ++b) {
                cur[b] = nxt[b];
                if constexpr (GATE) gcur[b] = gnxt[b];
            }
        }
    }

    reduce_rows<GATE, kWaves>(sh, acc, gacc, out, gout);
}

// The same partial sums for a short K range, by a workgroup of W waves: at
// most W*T groups (T tiles per wave; the range fits one LDS stage).  Every
// load is issued before the first wait: the activations first, so staging
// them waits for x only, then all of the wave's tiles (groups wave + W*i,
// clamped to the range; a clamped duplicate is loaded but never used).  The
// tiles then arrive in one overlapped window instead of one batch after
// another.
template <bool GATE, int T, int W, class Sh>
__device__ __forceinline__ void tile_row_partial_short(Sh &sh, const uint8_t *__restrict__ w,
                                                       const uint8_t *__restrict__ gw,
                                                       const float *__restrict__ x, uint32_t cols, uint32_t rt,
                                                       uint32_t g_begin, uint32_t g_end, float &out, float &gout,
                                                       PhaseClocks &clk) {
    static_assert(W * T <= static_cast<int>(sizeof(sh.st.c) / sizeof(sh.st.c[0])) &&
                      W <= static_cast<int>(sizeof(sh.red[0]) / sizeof(sh.red[0][0])),
                  "the range fits one stage");
    const uint32_t groups = cols / kGroup;
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int q = lane & 7, a = lane >> 3;
    const int ng = static_cast<int>(g_end - g_begin);
    const size_t first = (static_cast<size_t>(rt) * groups + g_begin) * kTileBytes;
    const uint8_t *wt = w + first;
    const uint8_t *gt = GATE ? gw + first : nullptr;

    // Thread t stages x items (group t/8 + 8Wm, lane slot t%8), m < XI.
    constexpr int XI = (T + 7) / 8;
    const int xa = threadIdx.x & 7;
    float l[XI][4], h[XI][4];
#pragma unroll
    for (int m = 0; m < XI; ++m) {
        const int xg = (threadIdx.x >> 3) + 8 * W * m;
#pragma unroll
        for (int j = 0; j < 4; ++j) l[m][j] = h[m][j] = 0.f;
        if (xg < ng) {
            const gptr_cf32 b = (gptr_cf32)x + (static_cast<size_t>(g_begin) + xg) * kGroup + 2 * xa;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                l[m][j] = b[16 * j];
                h[m][j] = b[16 * j + 1];
            }
        }
    }
    // Every wave's x loads are issued before any wave's tile loads (a bare
    // barrier, no wait for the loads): loads return in issue order, so
    // otherwise the last wave's x, which staging waits for, queues behind
    // the other waves' tiles.
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    TileRegs t[T], u[T];
#pragma unroll
    for (int i = 0; i < T; ++i) {
        const int gg = min(wave + W * i, ng - 1);
        t[i] = load_tile(wt + static_cast<size_t>(gg) * kTileBytes, q, a);
        if constexpr (GATE) u[i] = load_tile(gt + static_cast<size_t>(gg) * kTileBytes, q, a);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < XI; ++m) {
        const int xg = (threadIdx.x >> 3) + 8 * W * m;
        if (xg < ng) {
            const float *lm = l[m], *hm = h[m];
            sh.st.v[xg][xa] = make_float4(lm[0] * kEvenScale, lm[1] * kEvenScale, lm[2] * kEvenScale, lm[3] * kEvenScale);
            sh.st.v[xg][8 + xa] = make_float4(hm[0] * kOddScale, hm[1] * kOddScale, hm[2] * kOddScale, hm[3] * kOddScale);
            sh.st.c[xg][xa] = -8.0f * (((((((lm[0] + hm[0]) + lm[1]) + hm[1]) + lm[2]) + hm[2]) + lm[3]) + hm[3]);
        }
    }
    __syncthreads();
    phase_clock(clk, 1);
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    float gacc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < T; ++i) {
        const int gg = wave + W * i;
        if (gg < ng) {
            const float4 xl = sh.st.v[gg][a];
            const float4 xh = sh.st.v[gg][8 + a];
            const float c = sh.st.c[gg][a];
            tile_fma(t[i], xl, xh, c, acc);
            if constexpr (GATE) tile_fma(u[i], xl, xh, c, gacc);
        }
    }
    reduce_rows<GATE, W>(sh, acc, gacc, out, gout);
    phase_clock(clk, 2);
}

template <bool GATE, bool ADD>
__device__ __forceinline__ float epilogue(float v, float gv, const float *__restrict__ add, uint32_t row) {
    if constexpr (ADD) v += add[row];
    if constexpr (GATE) v *= silu(gv);
    return v;
}

// Where a row tile's chunk sums go (threads 0..31 hold row rt*32 + t's sum
// v and SwiGLU gate sum gv of chunk s): split 1 writes y; larger splits meet
// the row's other chunks in its exchange tree (exchange_tree), and the thread
// that clears the root applies the epilogue and writes y.  `add` may be null
// (ADD false makes it so at compile time).
template <bool GATE, bool ADD>
__device__ __forceinline__ void finish_rows(float *__restrict__ y, const float *__restrict__ add,
                                            uint32_t *__restrict__ slots, uint32_t rows, uint32_t split, uint32_t s,
                                            uint32_t rt, float v, float gv) {
    const uint32_t row = rt * kTileRows + (threadIdx.x & 31);
    if (threadIdx.x >= 32) return;
    // The bias is loaded before the exchanges, so its round trip overlaps
    // theirs instead of following the last one.
    float b = 0.f;
    if constexpr (ADD) b = add[row];
    if (split == 1 || exchange_tree<GATE>(slots, rows, split, s, row, v, gv)) {
        if constexpr (ADD) v += b;
        if constexpr (GATE) v *= silu(gv);
        y[row] = v;
    }
}

// Workgroup b covers row tile rt and K chunk s of `split`, remapped so the
// chunks of one row tile run on one XCD.
template <bool GATE, bool ADD, int T, int W>
__global__ __launch_bounds__(64 * W) void gemv_kernel(GemvArgs args) {
    __shared__ SharedFor<W> sh;
    PhaseClocks clk;
    phase_clock(clk, 0);
    const uint32_t groups = args.cols / kGroup;
    const uint32_t split = args.split;
    const uint32_t logical = xcd_remap(blockIdx.x, gridDim.x);
    const uint32_t rt = div_split(logical, split, args.split_magic), s = logical - rt * split;
    const uint32_t g_begin = div_split(s * groups, split, args.split_magic);
    const uint32_t g_end = div_split((s + 1) * groups, split, args.split_magic);
    float v = 0.f, gv = 0.f;
    if constexpr (T == 0)
        tile_row_partial<GATE>(sh, args.w, args.gate, args.x, args.cols, rt, g_begin, g_end, v, gv);
    else
        tile_row_partial_short<GATE, T, W>(sh, args.w, args.gate, args.x, args.cols, rt, g_begin, g_end, v, gv, clk);
    finish_rows<GATE, ADD>(args.y, args.add, args.slots, args.rows, split, s, rt, v, gv);
    if constexpr (T != 0) phase_record(clk, args.clock_slot);
}

// Several GEMVs sharing x (q4rdna_mul_mat_group): the row tiles of all of
// them form one index space, GEMV i owning [tile_begin_i, tile_begin_i +
// rows_i / 32); workgroup b covers one (row tile, K chunk) as gemv_kernel
// does.  Every K chunk holds at most W*T groups (the short-range path).
template <bool GATE, int T, int W>
__global__ __launch_bounds__(64 * W) void gemv_group_kernel(GemvGroupArgs a) {
    __shared__ Shared sh;
    PhaseClocks clk;
    phase_clock(clk, 0);
    const uint32_t groups = a.cols / kGroup;
    const uint32_t split = a.split;
    const uint32_t logical = xcd_remap(blockIdx.x, gridDim.x);
    const uint32_t gt = div_split(logical, split, a.split_magic), s = logical - gt * split;
    // The workgroup's GEMV (constant indices only, so the entries stay in
    // the kernel-argument segment).
    GemvGroupEntry G = a.g[0];
#pragma unroll
    for (uint32_t i = 1; i < kMaxGroup; ++i)
        if (i < a.count && gt >= a.g[i].tile_begin) G = a.g[i];
    const uint32_t rt = gt - G.tile_begin;
    const uint32_t g_begin = div_split(s * groups, split, a.split_magic);
    const uint32_t g_end = div_split((s + 1) * groups, split, a.split_magic);
    float v = 0.f, gv = 0.f;
    tile_row_partial_short<GATE, T, W>(sh, G.w, G.gate, a.x, a.cols, rt, g_begin, g_end, v, gv, clk);
    if (G.add != nullptr)
        finish_rows<GATE, true>(G.y, G.add, G.slots, G.rows, split, s, rt, v, gv);
    else
        finish_rows<GATE, false>(G.y, nullptr, G.slots, G.rows, split, s, rt, v, gv);
    phase_record(clk, a.clock_slot);
}

// ---- several activation vectors against one weight (n = 2..8) -------------
//
// The short-range kernel above with NV vector slots (n <= NV used): x is
// [n][cols], y and add are [n][rows].  Each tile is loaded and decoded once
// and applied to every vector, so a launch costs about what one vector does
// while it is latency-bound.  Every step of a vector's arithmetic and
// summation is the one-vector kernel's (same x staging, same fma order, same
// lane, wave and chunk order), so each vector's result is bit-identical to
// q4rdna_mul_mat_ex of that vector with the same split and eight waves.
constexpr int kMvWaves = 8;

// Groups one workgroup stages: NV vectors' x fit 37 KB of LDS.
template <int NV>
constexpr int mv_stage_groups() { return NV >= 8 ? 16 : 32; }

template <int NV>
struct MvShared {
    float4 v[NV][mv_stage_groups<NV>()][16];  // [vector][g][a] even-k x, [..][8 + a] odd-k x / 16
    float c[NV][mv_stage_groups<NV>()][8];    // -8 * sum of the lane's 8 x values
    float red[2][NV][kMvWaves][32];
};

template <bool GATE, bool ADD, int NV, int T>
__global__ __launch_bounds__(64 * kMvWaves) void gemv_multi_kernel(GemvArgs args) {
    constexpr int W = kMvWaves;
    constexpr int SG = mv_stage_groups<NV>();
    static_assert(W * T <= SG, "a chunk fits the stage");
    __shared__ MvShared<NV> sh;
    const uint32_t groups = args.cols / kGroup;
    const uint32_t split = args.split;
    const uint32_t nv = args.vectors;
    const uint32_t logical = xcd_remap(blockIdx.x, gridDim.x);
    const uint32_t rt = div_split(logical, split, args.split_magic), s = logical - rt * split;
    const uint32_t g_begin = div_split(s * groups, split, args.split_magic);
    const uint32_t g_end = div_split((s + 1) * groups, split, args.split_magic);
    const int ng = static_cast<int>(g_end - g_begin);
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int q = lane & 7, a = lane >> 3;
    const size_t first = (static_cast<size_t>(rt) * groups + g_begin) * kTileBytes;
    const uint8_t *wt = args.w + first;
    const uint8_t *gt = GATE ? args.gate + first : nullptr;

    // Activations first (item = (vector, group, lane slot), thread t takes
    // items t + 64W*m), then every tile of the wave, then the x staging.
    constexpr int XI = (NV * SG * 8 + 64 * W - 1) / (64 * W);
    float l[XI][4], h[XI][4];
#pragma unroll
    for (int m = 0; m < XI; ++m) {
        const int item = threadIdx.x + 64 * W * m;
        const int v = item / (SG * 8), xg = (item >> 3) % SG, xa = item & 7;
#pragma unroll
        for (int j = 0; j < 4; ++j) l[m][j] = h[m][j] = 0.f;
        if (v < static_cast<int>(nv) && xg < ng) {
            const gptr_cf32 b = (gptr_cf32)args.x + static_cast<size_t>(v) * args.cols +
                                (static_cast<size_t>(g_begin) + xg) * kGroup + 2 * xa;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                l[m][j] = b[16 * j];
                h[m][j] = b[16 * j + 1];
            }
        }
    }
    // Every wave's x loads are issued before any wave's tile loads (a bare
    // barrier, no wait for the loads): loads return in issue order, so
    // otherwise the last wave's x, which staging waits for, queues behind
    // the other waves' tiles.
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    TileRegs t[T], u[T];
#pragma unroll
    for (int i = 0; i < T; ++i) {
        const int gg = min(wave + W * i, ng - 1);
        t[i] = load_tile(wt + static_cast<size_t>(gg) * kTileBytes, q, a);
        if constexpr (GATE) u[i] = load_tile(gt + static_cast<size_t>(gg) * kTileBytes, q, a);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < XI; ++m) {
        const int item = threadIdx.x + 64 * W * m;
        const int v = item / (SG * 8), xg = (item >> 3) % SG, xa = item & 7;
        if (v < static_cast<int>(nv) && xg < ng) {
            const float *lm = l[m], *hm = h[m];
            sh.v[v][xg][xa] = make_float4(lm[0] * kEvenScale, lm[1] * kEvenScale, lm[2] * kEvenScale, lm[3] * kEvenScale);
            sh.v[v][xg][8 + xa] = make_float4(hm[0] * kOddScale, hm[1] * kOddScale, hm[2] * kOddScale, hm[3] * kOddScale);
            sh.c[v][xg][xa] = -8.0f * (((((((lm[0] + hm[0]) + lm[1]) + hm[1]) + lm[2]) + hm[2]) + lm[3]) + hm[3]);
        }
    }
    __syncthreads();

    float acc[NV][4], gacc[NV][4];
#pragma unroll
    for (int v = 0; v < NV; ++v)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[v][r] = gacc[v][r] = 0.f;
#pragma unroll
    for (int i = 0; i < T; ++i) {
        const int gg = wave + W * i;
        if (gg < ng) {
            const TileCodes w = split_codes(t[i].d);
            TileCodes gw;
            if constexpr (GATE) gw = split_codes(u[i].d);
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                if (v < static_cast<int>(nv)) {
                    const float4 xl = sh.v[v][gg][a];
                    const float4 xh = sh.v[v][gg][8 + a];
                    const float c = sh.c[v][gg][a];
                    apply_codes(w, t[i].s01, t[i].s23, xl, xh, c, acc[v]);
                    if constexpr (GATE) apply_codes(gw, u[i].s01, u[i].s23, xl, xh, c, gacc[v]);
                }
            }
        }
    }

    // Lanes, then waves in wave order (reduce_rows, per vector).
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        const float tot = add_over_a4(acc[v]);
        float gtot = 0.f;
        if constexpr (GATE) gtot = add_over_a4(gacc[v]);
        if ((lane & 8) == 0) {
            const int row = 4 * (lane & 7) + (lane >> 4);
            sh.red[0][v][wave][row] = tot;
            if constexpr (GATE) sh.red[1][v][wave][row] = gtot;
        }
    }
    __syncthreads();
    // Thread t < 32*nv finishes row t % 32 of vector t / 32.
    const uint32_t v = threadIdx.x >> 5, rl = threadIdx.x & 31;
    const bool mine = v < nv;
    const uint32_t row = rt * kTileRows + rl;
    const size_t M = args.rows;
    float out = 0.f, gout = 0.f;
    if (mine) {
        out = sh.red[0][v][0][rl];
#pragma unroll
        for (int wv = 1; wv < W; ++wv) out += sh.red[0][v][wv][rl];
        if constexpr (GATE) {
            gout = sh.red[1][v][0][rl];
#pragma unroll
            for (int wv = 1; wv < W; ++wv) gout += sh.red[1][v][wv][rl];
        }
    }
    // Split K as in gemv_kernel: an exchange tree per (vector, row), each
    // node's region holding [vector][rows] slots.
    if (mine && (split == 1 || exchange_tree<GATE>(args.slots, nv * static_cast<uint32_t>(M), split, s,
                                                   v * static_cast<uint32_t>(M) + row, out, gout)))
        args.y[v * M + row] = epilogue<GATE, ADD>(out, gout, args.add ? args.add + v * M : nullptr, row);
}

// The reference's old mapping (source/q4rdna.cu:190-234, selected there by
// LLAMA_Q4_RDNA_MAPPING=old): one thread per row, its weights in k order,
// one fp32 fma each, sum = fma(scale * q, x_k, sum) -- the CPU loop's
// arithmetic step for step, so the result is its bits.  x is staged one
// group at a time in LDS; rows past the end compute a stand-in row and
// store nothing (every thread reaches the barriers).
constexpr int kSeqThreads = 256;
template <bool GATE, bool ADD>
__global__ __launch_bounds__(kSeqThreads) void gemv_sequential_kernel(GemvArgs args) {
    __shared__ float xs[kGroup];
    const uint32_t groups = args.cols / kGroup;
    const uint32_t row = blockIdx.x * kSeqThreads + threadIdx.x;
    const uint32_t r = min(row, args.rows - 1);
    const uint32_t rt = r / kTileRows, lane = r % kTileRows;
    const uint8_t *wt = args.w + static_cast<size_t>(rt) * groups * kTileBytes;
    const uint8_t *gt = GATE ? args.gate + static_cast<size_t>(rt) * groups * kTileBytes : nullptr;
    float sum = 0.f, gsum = 0.f;
    for (uint32_t g = 0; g < groups; ++g) {
        __syncthreads();
        if (threadIdx.x < kGroup) xs[threadIdx.x] = args.x[static_cast<size_t>(g) * kGroup + threadIdx.x];
        __syncthreads();
        const uint8_t *tile = wt + static_cast<size_t>(g) * kTileBytes;
        const float scale = half_bits_to_float(tile[2 * lane] | (static_cast<uint32_t>(tile[2 * lane + 1]) << 8));
        float gscale = 0.f;
        if constexpr (GATE)
            gscale = half_bits_to_float(gt[static_cast<size_t>(g) * kTileBytes + 2 * lane] |
                                        (static_cast<uint32_t>(gt[static_cast<size_t>(g) * kTileBytes + 2 * lane + 1]) << 8));
        for (int i = 0; i < static_cast<int>(kGroup / 2); ++i) {
            const uint8_t b = tile[64 + kTileRows * i + lane];
            const int lo = static_cast<int>(static_cast<int8_t>(static_cast<uint8_t>(b << 4))) >> 4;
            const int hi = static_cast<int>(static_cast<int8_t>(b)) >> 4;
            sum = fmaf(scale * static_cast<float>(lo), xs[2 * i], sum);
            sum = fmaf(scale * static_cast<float>(hi), xs[2 * i + 1], sum);
            if constexpr (GATE) {
                const uint8_t gb = gt[static_cast<size_t>(g) * kTileBytes + 64 + kTileRows * i + lane];
                const int glo = static_cast<int>(static_cast<int8_t>(static_cast<uint8_t>(gb << 4))) >> 4;
                const int ghi = static_cast<int>(static_cast<int8_t>(gb)) >> 4;
                gsum = fmaf(gscale * static_cast<float>(glo), xs[2 * i], gsum);
                gsum = fmaf(gscale * static_cast<float>(ghi), xs[2 * i + 1], gsum);
            }
        }
    }
    if (row < args.rows) args.y[row] = epilogue<GATE, ADD>(sum, gsum, args.add, row);
}

// out[row][k] = fp32(scale) * code, one thread per code byte.
__global__ __launch_bounds__(kThreads) void dequant_kernel(const uint8_t *__restrict__ w, uint32_t rows,
                                                           uint32_t cols, float *__restrict__ out) {
    const uint32_t groups = cols / kGroup;
    const uint64_t total = static_cast<uint64_t>(rows) * cols / 2;
    for (uint64_t idx = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
         idx += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        const uint64_t t = idx >> 10;
        const uint32_t rem = static_cast<uint32_t>(idx & 1023u);
        const uint32_t i = rem >> 5, l = rem & 31u;
        const uint64_t rt = t / groups, g = t % groups;
        const uint8_t *tile = w + t * kTileBytes;
        const float scale = half_bits_to_float(tile[2 * l] | (static_cast<uint32_t>(tile[2 * l + 1]) << 8));
        const uint8_t b = tile[64 + rem];
        const int lo = static_cast<int>(static_cast<int8_t>(static_cast<uint8_t>(b << 4))) >> 4;
        const int hi = static_cast<int>(static_cast<int8_t>(b)) >> 4;
        const uint64_t row = rt * kTileRows + l;
        const uint64_t k = g * kGroup + 2 * i;
        out[row * cols + k] = scale * static_cast<float>(lo);
        out[row * cols + k + 1] = scale * static_cast<float>(hi);
    }
}

// ---------------------------------------------------------------------------
// Packer: one thread per (row, group), bit-identical to the reference CPU
// packers (source/q4rdna_sidecar_pack.cpp:126-179, 259-279 and
// source/q4rdna_cpu_experiment.cpp:136-273, 387-399).  Bit-identical output
// fixes the arithmetic: every sum runs in index order, contraction is off so
// each product and sum rounds on its own, '/' is the correctly rounded IEEE
// division, and rintf ties to even like nearbyint under FE_TONEAREST.
// ---------------------------------------------------------------------------
#pragma clang fp contract(off)

// The reference tools' binary16 conversions, by their behaviour, on the
// hardware conversions.  Encode: IEEE round to nearest even, except that NaN
// becomes an infinity of its sign.  Decode: exact, except that a subnormal
// comes out at half its value (their normalisation uses a normal number's
// exponent bias).  The scale search runs on this decode, so the packed bytes
// depend on it; the GEMV and dequant kernels decode scales exactly, as the
// reference's GPU kernels do (__half2float).
__device__ __forceinline__ uint32_t packer_encode(float v) {
    if (isnan(v)) return ((__float_as_uint(v) >> 16) & 0x8000u) | 0x7c00u;
    return __half_as_ushort(__float2half_rn(v));
}

__device__ __forceinline__ float packer_decode(uint32_t h) {
    const float exact = half_bits_to_float(h);
    return ((h & 0x7c00u) == 0u && (h & 0x03ffu) != 0u) ? 0.5f * exact : exact;
}

// int(t) of an integral float as x86-64 converts it (INT_MIN when out of
// range), the conversion the reference tools' int(...) made where they ran.
__device__ __forceinline__ int to_int_x86(float t) {
    if (!(t >= -2147483648.0f && t < 2147483648.0f)) return static_cast<int>(0x80000000u);
    return static_cast<int>(t);
}

// Code of v at scale s: v / s rounded (ties to even for the sidecar packer,
// away from zero for the CPU experiment), clamped to [-8, 7]; 0 at s = 0.
template <bool TIES_EVEN>
__device__ __forceinline__ int code_at(float v, float s) {
    if (s == 0.0f) return 0;
    const float r = TIES_EVEN ? rintf(v / s) : roundf(v / s);
    const int c = to_int_x86(r);
    return c < -8 ? -8 : (c > 7 ? 7 : c);
}

// A group's extremes and the two "range" scales that map them onto the code
// range: the positive one puts max v at +7 or min v at -8, whichever needs
// the larger scale; the negative one mirrors it.  The running maxima start
// at 0 and keep the old value unless the new one is strictly larger (a NaN
// never replaces anything).
struct GroupRange {
    float pos_max, neg_max, abs_max;
    float pos_scale, neg_scale;
};

__device__ __forceinline__ float keep_larger(float a, float b) { return a < b ? b : a; }

__device__ GroupRange group_range(const float *v) {
    GroupRange g{0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = 0; i < 64; ++i) {
        g.pos_max = keep_larger(g.pos_max, v[i]);
        g.neg_max = keep_larger(g.neg_max, -v[i]);
        g.abs_max = keep_larger(g.abs_max, fabsf(v[i]));
    }
    g.pos_scale = keep_larger(g.pos_max / 7.0f, g.neg_max / 8.0f);
    g.neg_scale = -keep_larger(g.pos_max / 8.0f, g.neg_max / 7.0f);
    return g;
}

// The sidecar packer's sums at one scale, in fp32: the squared error of the
// codes and the least-squares terms sum v*q and sum q*q of a refit.  One pass
// computes all three from the same codes; each sum keeps index order.
struct FitF32 {
    float err, num, den;
};

__device__ FitF32 fit_f32(const float *v, float s) {
    FitF32 f{0.0f, 0.0f, 0.0f};
    for (int i = 0; i < 64; ++i) {
        const int q = code_at<true>(v[i], s);
        const float d = s * static_cast<float>(q) - v[i];
        f.err += d * d;
        f.num += v[i] * static_cast<float>(q);
        f.den += static_cast<float>(q * q);
    }
    return f;
}

// Sidecar search: ten starts (the positive and the negative range scale,
// times 1, 0.9, 0.8, 0.7, 0.6, positive first at each factor), each refitted
// by least squares until its fp16 scale repeats, for at most 12 evaluations;
// the scale of least error wins, the earliest on ties.  An all-zero group
// gets scale 0.
__device__ uint32_t search_sidecar(const float *v) {
    const GroupRange g = group_range(v);
    if (g.pos_max == 0.0f && g.neg_max == 0.0f) return 0;
    const float factor[5] = {1.0f, 0.9f, 0.8f, 0.7f, 0.6f};
    uint32_t best = 0;
    float best_err = __builtin_huge_valf();
    for (int start = 0; start < 10; ++start) {
        uint32_t h = packer_encode(((start & 1) ? g.neg_scale : g.pos_scale) * factor[start >> 1]);
        for (int eval = 0; eval < 12; ++eval) {
            const FitF32 f = fit_f32(v, packer_decode(h));
            if (f.err < best_err) {
                best_err = f.err;
                best = h;
            }
            if (f.den == 0.0f) break;
            const uint32_t next = packer_encode(f.num / f.den);
            if (next == h) break;
            h = next;
        }
    }
    return best;
}

// The CPU experiment's bookkeeping: the best fp16 scale so far and its
// squared error in double.
struct Best {
    double err;
    uint32_t bits;
};

// Squared error, in double, of the codes (ties away from zero) at scale s.
__device__ double err_f64(const float *v, float s) {
    double e = 0.0;
    for (int i = 0; i < 64; ++i) {
        const double d = static_cast<double>(s) * static_cast<double>(code_at<false>(v[i], s)) - static_cast<double>(v[i]);
        e += d * d;
    }
    return e;
}

// Offer scale s: a finite s is stored as fp16 and judged at the value those
// bits decode to; it replaces the best if its error is strictly smaller.
__device__ void offer(const float *v, float s, Best &b) {
    if (!isfinite(s)) return;
    const uint32_t h = packer_encode(s);
    const double e = err_f64(v, packer_decode(h));
    if (e < b.err) {
        b.err = e;
        b.bits = h;
    }
}

// One start of the experiment's mse search: up to 12 least-squares refits in
// double, each offered, stopping when the fp16 scale repeats or every code is
// zero; then the two fp16 magnitudes adjacent to the best so far.
__device__ void refit_f64(const float *v, float s0, Best &b) {
    uint32_t h = packer_encode(s0);
    for (int eval = 0; eval < 12; ++eval) {
        const float s = packer_decode(h);
        offer(v, s, b);
        double num = 0.0, den = 0.0;
        for (int i = 0; i < 64; ++i) {
            const double q = static_cast<double>(code_at<false>(v[i], s));
            num += static_cast<double>(v[i]) * q;
            den += q * q;
        }
        if (den == 0.0) break;
        const uint32_t next = packer_encode(static_cast<float>(num / den));
        if (next == h) break;
        h = next;
    }
    const uint32_t mag = b.bits & 0x7fffu, sign = b.bits & 0x8000u;
    if (mag != 0u && mag < 0x7bffu) {
        offer(v, packer_decode(sign | (mag - 1u)), b);
        offer(v, packer_decode(sign | (mag + 1u)), b);
    }
}

// The CPU experiment's three searches: absmax = fp16(max|v| / 7); range =
// the better of the two range scales; mse = range, then 24 refitted starts
// (the two range scales times 1 .. 0.25, positive first at each factor).
__device__ uint32_t search_experiment(const float *v, int algorithm) {
    const GroupRange g = group_range(v);
    if (g.abs_max == 0.0f) return 0;
    if (algorithm == 1) return packer_encode(g.abs_max / 7.0f);
    Best b{__builtin_huge_val(), 0u};
    offer(v, g.pos_scale, b);
    offer(v, g.neg_scale, b);
    if (algorithm == 2) return b.bits;
    const float factor[12] = {1.0f, 0.9f, 0.8f, 0.7f, 0.6f, 0.55f, 0.5f, 0.45f, 0.4f, 0.35f, 0.3f, 0.25f};
    for (int start = 0; start < 24; ++start)
        refit_f64(v, ((start & 1) ? g.neg_scale : g.pos_scale) * factor[start >> 1], b);
    return b.bits;
}

// Thread per (row, group) ordered (row tile, group, row lane) so a wave's
// scale and code stores land in contiguous bytes of one tile.
__global__ __launch_bounds__(kThreads) void pack_kernel(const float *__restrict__ w, uint32_t rows,
                                                        uint32_t cols, int algorithm,
                                                        uint8_t *__restrict__ tiles) {
    const uint32_t groups = cols / kGroup;
    const uint64_t total = static_cast<uint64_t>(rows) * groups;
    for (uint64_t idx = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
         idx += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        const uint64_t t = idx >> 5;
        const uint32_t l = static_cast<uint32_t>(idx & 31u);
        const uint64_t rt = t / groups, g = t % groups;
        const uint64_t row = rt * kTileRows + l;
        float v[64];
        const float4 *src = reinterpret_cast<const float4 *>(w + row * cols + g * kGroup);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float4 f = src[i];
            v[4 * i] = f.x;
            v[4 * i + 1] = f.y;
            v[4 * i + 2] = f.z;
            v[4 * i + 3] = f.w;
        }
        const uint32_t bits = algorithm == 0 ? search_sidecar(v) : search_experiment(v, algorithm);
        const float scale = packer_decode(bits);
        uint8_t *tile = tiles + t * kTileBytes;
        tile[2 * l] = static_cast<uint8_t>(bits & 0xffu);
        tile[2 * l + 1] = static_cast<uint8_t>(bits >> 8);
        for (int i = 0; i < 32; ++i) {
            const int lo = algorithm == 0 ? code_at<true>(v[2 * i], scale) : code_at<false>(v[2 * i], scale);
            const int hi = algorithm == 0 ? code_at<true>(v[2 * i + 1], scale) : code_at<false>(v[2 * i + 1], scale);
            tile[64 + 32 * i + l] = static_cast<uint8_t>((lo & 15) | ((hi & 15) << 4));
        }
    }
}

#pragma clang fp contract(on)

// K chunks of at most 64 groups run the short-range kernel with W = 8 or 4
// waves (args.short_waves) and T <= 64 / W tiles per wave; chunks of up to
// 128 groups the wide workgroup of 16 waves and T <= 8; longer chunks the
// pipelined loop (T = 0) with kWaves waves.  The host keeps split <= groups,
// so every chunk holds at least one group.
template <bool GATE, bool ADD, int W>
hipError_t launch_gemv_w(const GemvArgs &args, hipStream_t stream) {
    const uint32_t blocks = (args.rows / kTileRows) * args.split;
    const uint32_t groups = args.cols / kGroup;
    const uint32_t per_wave = ((groups + args.split - 1) / args.split + W - 1) / W;
    const dim3 grid(blocks), block(64 * W);
    if constexpr (W == kWideWaves) {
        if (per_wave <= 4)
            hipLaunchKernelGGL((gemv_kernel<GATE, ADD, 4, W>), grid, block, 0, stream, args);
        else if (per_wave <= 6)
            hipLaunchKernelGGL((gemv_kernel<GATE, ADD, 6, W>), grid, block, 0, stream, args);
        else if (per_wave <= 8)
            hipLaunchKernelGGL((gemv_kernel<GATE, ADD, 8, W>), grid, block, 0, stream, args);
        else
            return hipErrorInvalidValue;
        return hipGetLastError();
    } else if (per_wave <= 1)
        hipLaunchKernelGGL((gemv_kernel<GATE, ADD, 1, W>), grid, block, 0, stream, args);
    else if (per_wave <= 2)
        hipLaunchKernelGGL((gemv_kernel<GATE, ADD, 2, W>), grid, block, 0, stream, args);
    else if (per_wave <= 4)
        hipLaunchKernelGGL((gemv_kernel<GATE, ADD, 4, W>), grid, block, 0, stream, args);
    else if (per_wave <= 8)
        hipLaunchKernelGGL((gemv_kernel<GATE, ADD, 8, W>), grid, block, 0, stream, args);
    else if (W == 4 && per_wave <= 16)
        hipLaunchKernelGGL((gemv_kernel<GATE, ADD, 64 / W, W>), grid, block, 0, stream, args);
    else
        hipLaunchKernelGGL((gemv_kernel<GATE, ADD, 0, kWaves>), grid, dim3(kThreads), 0, stream, args);
    return hipGetLastError();
}

template <bool GATE, bool ADD>
hipError_t launch_gemv_t(const GemvArgs &args, hipStream_t stream) {
    if (args.short_waves == kWideWaves) return launch_gemv_w<GATE, ADD, kWideWaves>(args, stream);
    return args.short_waves == kShortWaves ? launch_gemv_w<GATE, ADD, kShortWaves>(args, stream)
                                           : launch_gemv_w<GATE, ADD, kWaves>(args, stream);
}

template <bool GATE, bool ADD, int NV>
hipError_t launch_multi_nv(const GemvArgs &args, hipStream_t stream) {
    constexpr int W = kMvWaves;
    const uint32_t blocks = (args.rows / kTileRows) * args.split;
    const uint32_t groups = args.cols / kGroup;
    const uint32_t per_wave = ((groups + args.split - 1) / args.split + W - 1) / W;
    const dim3 grid(blocks), block(64 * W);
    if (per_wave <= 1)
        hipLaunchKernelGGL((gemv_multi_kernel<GATE, ADD, NV, 1>), grid, block, 0, stream, args);
    else if (per_wave <= 2 || NV >= 8)
        hipLaunchKernelGGL((gemv_multi_kernel<GATE, ADD, NV, 2>), grid, block, 0, stream, args);
    else
        hipLaunchKernelGGL((gemv_multi_kernel<GATE, ADD, NV, (NV >= 8 ? 2 : 4)>), grid, block, 0, stream, args);
    return hipGetLastError();
}

template <bool GATE, bool ADD>
hipError_t launch_multi_t(const GemvArgs &args, hipStream_t stream) {
    if (args.vectors <= 2) return launch_multi_nv<GATE, ADD, 2>(args, stream);
    if (args.vectors <= 4) return launch_multi_nv<GATE, ADD, 4>(args, stream);
    return launch_multi_nv<GATE, ADD, 8>(args, stream);
}

uint32_t grid_for(uint64_t work, uint32_t per_block) {
    uint64_t blocks = (work + per_block - 1) / per_block;
    if (blocks > 65536) blocks = 65536;
    return static_cast<uint32_t>(blocks == 0 ? 1 : blocks);
}

}  // namespace

hipError_t launch_gemv(const GemvArgs &args, hipStream_t stream) {
    if (args.gate != nullptr) {
        return args.add != nullptr ? launch_gemv_t<true, true>(args, stream)
                                   : launch_gemv_t<true, false>(args, stream);
    }
    return args.add != nullptr ? launch_gemv_t<false, true>(args, stream)
                               : launch_gemv_t<false, false>(args, stream);
}

hipError_t launch_gemv_group(const GemvGroupArgs &args, hipStream_t stream) {
    const uint32_t groups = args.cols / kGroup;
    const uint32_t chunk = (groups + args.split - 1) / args.split;
    const dim3 grid(args.tiles * args.split);
    const bool glu = args.g[0].gate != nullptr;
    auto go = [&](auto gate_tag, auto t_tag, auto w_tag) {
        constexpr bool G = decltype(gate_tag)::value;
        constexpr int T = decltype(t_tag)::value, W = decltype(w_tag)::value;
        hipLaunchKernelGGL((gemv_group_kernel<G, T, W>), grid, dim3(64 * W), 0, stream, args);
    };
    using F = std::false_type;
    using Tr = std::true_type;
    auto by_t = [&](auto gate_tag, auto w_tag) {
        constexpr int W = decltype(w_tag)::value;
        const uint32_t per_wave = (chunk + W - 1) / W;
        if (per_wave <= 1) go(gate_tag, std::integral_constant<int, 1>{}, w_tag);
        else if (per_wave <= 2) go(gate_tag, std::integral_constant<int, 2>{}, w_tag);
        else if (per_wave <= 4) go(gate_tag, std::integral_constant<int, 4>{}, w_tag);
        else if (per_wave <= 8) go(gate_tag, std::integral_constant<int, 8>{}, w_tag);
        else go(gate_tag, std::integral_constant<int, 64 / W>{}, w_tag);
    };
    if (args.short_waves == kShortWaves) {
        if (glu) by_t(Tr{}, std::integral_constant<int, kShortWaves>{});
        else by_t(F{}, std::integral_constant<int, kShortWaves>{});
    } else {
        if (glu) by_t(Tr{}, std::integral_constant<int, kWaves>{});
        else by_t(F{}, std::integral_constant<int, kWaves>{});
    }
    return hipGetLastError();
}

hipError_t launch_gemv_multi(const GemvArgs &args, hipStream_t stream) {
    if (args.gate != nullptr) {
        return args.add != nullptr ? launch_multi_t<true, true>(args, stream)
                                   : launch_multi_t<true, false>(args, stream);
    }
    return args.add != nullptr ? launch_multi_t<false, true>(args, stream)
                               : launch_multi_t<false, false>(args, stream);
}

hipError_t launch_gemv_sequential(const GemvArgs &args, hipStream_t stream) {
    const dim3 grid((args.rows + kSeqThreads - 1) / kSeqThreads), block(kSeqThreads);
    if (args.gate != nullptr) {
        if (args.add != nullptr) hipLaunchKernelGGL((gemv_sequential_kernel<true, true>), grid, block, 0, stream, args);
        else hipLaunchKernelGGL((gemv_sequential_kernel<true, false>), grid, block, 0, stream, args);
    } else {
        if (args.add != nullptr) hipLaunchKernelGGL((gemv_sequential_kernel<false, true>), grid, block, 0, stream, args);
        else hipLaunchKernelGGL((gemv_sequential_kernel<false, false>), grid, block, 0, stream, args);
    }
    return hipGetLastError();
}

uint32_t gemv_multi_stage_groups(uint32_t vectors) { return vectors > 4 ? 16u : 32u; }

uint32_t gemv_waves(uint32_t groups, uint32_t split, uint64_t workgroups, uint32_t cus) {
    const uint32_t chunk = (groups + split - 1) / split;
    // A chunk longer than one eight-wave stage runs on 16 waves (one
    // workgroup per CU, every tile in flight) while it fits their registers.
    if (chunk > static_cast<uint32_t>(kStageGroups) && chunk <= static_cast<uint32_t>(kWideStageGroups) &&
        workgroups <= cus)
        return kWideWaves;
    // Eight waves per workgroup while the launch is latency-bound (at most
    // four workgroups per CU); with more, four waves of up to 16 tiles keep
    // more bytes in flight per CU (151936x4096: 60 us against 68).
    return workgroups <= 4ull * cus ? kShortWaves : kWaves;
}

hipError_t launch_dequant(const uint8_t *w, uint32_t rows, uint32_t cols, float *out, hipStream_t stream) {
    const uint64_t work = static_cast<uint64_t>(rows) * cols / 2;
    hipLaunchKernelGGL(dequant_kernel, dim3(grid_for(work, kThreads)), dim3(kThreads), 0, stream, w, rows,
                       cols, out);
    return hipGetLastError();
}

hipError_t launch_pack(const float *w, uint32_t rows, uint32_t cols, int algorithm, uint8_t *tiles,
                       hipStream_t stream) {
    const uint64_t work = static_cast<uint64_t>(rows) * (cols / kGroup);
    hipLaunchKernelGGL(pack_kernel, dim3(grid_for(work, kThreads)), dim3(kThreads), 0, stream, w, rows, cols,
                       algorithm, tiles);
    return hipGetLastError();
}

}  // namespace q4rdna

#if defined(Q4RDNA_SWEEP_CLOCKS)
// Clock build only: the record of launch slot `slot`, kGemvClockWords words
// for each of workgroups 0..count-1 (count <= kGemvClockWorkgroups).
extern "C" int q4rdna_gemv_clocks(uint32_t slot, uint64_t *out, uint32_t count) {
    if (out == nullptr || slot >= q4rdna::kGemvClockSlots || count > q4rdna::kGemvClockWorkgroups) return -1;
    const size_t words = q4rdna::kGemvClockWords;
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(q4rdna::g_gemv_clocks), words * sizeof(uint64_t) * count,
                               words * sizeof(uint64_t) * q4rdna::kGemvClockWorkgroups * slot,
                               hipMemcpyDeviceToHost) == hipSuccess ? 0 : -4;
}
#endif
