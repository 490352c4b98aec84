// gfx950 int8-MFMA path of the Q4_RDNA GEMV (multi-tensor plans).
//
// The VALU path spends one conversion and one fma per weight.  Here the
// multiply-accumulate runs on the matrix cores instead, with exact integer
// arithmetic:
//
//  * Codes.  A code byte holds two's-complement nibbles q(2i) (low) and
//    q(2i+1) (high).  (b << 4) & 0xF0 and b & 0xF0 are the int8 values
//    16*q(2i) and 16*q(2i+1), so a dword of four code bytes becomes two int8x4
//    operand dwords with one shift and two masks.
//
//  * Activations.  Each 64-element group of x is written as block floating
//    point: E = the exponent of max|x| (frexp), A_k = rint(x_k * 2^(22-E))
//    (|A_k| <= 2^22), split into three balanced int8 digits
//    A = a0 + 256*a1 + 65536*a2.  x_k = A_k * 2^(E-22) to within 2^-23 of the
//    group maximum, so the GEMV keeps fp32-level accuracy.
//
//  * v_mfma_i32_16x16x64_i8: D[i][j] = sum_k A[i][k] B[k][j] with A = the three
//    digit rows of x (row 3 zero) and B = 16 weight rows, one group (64 k) per
//    instruction; |D| <= 64 * 128 * 128 = 2^20, exact in int32.  Lane l
//    supplies A row l%16 and B column l%16 for k-slot l/16 (16 bytes each) and
//    receives D[4*(l/16) + v][l%16] -- checked on the device against a CPU
//    product.  Per (row, group) the result is
//    scale * 2^(E-26) * (D0 + 256*D1 + 65536*D2) (2^-4 undoes the 16*q).
//
//  * Layout.  A wave takes a 64-row block (two 32-row tiles) and one group per
//    step.  Lane (kslot = l/16, j = l%16) loads, from tile j/8, the eight code
//    dwords of rows 4(j%8)..+3 at k-pairs 4c + kslot, c = 0..7 (so each load
//    instruction reads 128 contiguous bytes of each tile), transposes the two
//    4x4 byte blocks (c = 0..3, 4..7) with v_perm_b32 so each dword holds one
//    row's four k-pairs, and splits nibbles: the four B operands of rows
//    4j+0..3 for four MFMAs.  Element e of a lane's operand is
//    k = 2*(16*(e/8) + 4*(e%4) + kslot) + (e/4)%2 within the group; the
//    activation digits are stored in the same order.
//
// About 38 VALU instructions per 2048-weight tile instead of ~99.
#include "q4rdna_device.h"

namespace q4rdna {
namespace {

constexpr int kWaves = 4;

// Position of element k (0..63) of a group in the operand order above:
// returns the byte index e (0..15) and the k-slot.
__device__ __forceinline__ int operand_index(int k, int &kslot) {
    const int i = k >> 1, h = k & 1;
    kslot = i & 3;
    const int c = i >> 2;
    return 4 * (2 * (c >> 2) + h) + (c & 3);
}

// One wave per 64-element activation group: block exponent, three int8
// digits per element in operand order, and the group factor 2^(E-26).
// Prep layout per group (kPrepBytes = 272): byte (kslot*4 + digit)*16 + e for
// digit 0..2, digit slot 3 zero; float factor at 256; zero padding to 272.
__global__ __launch_bounds__(256) void prep_kernel(const PlanDesc *__restrict__ descs, uint32_t count,
                                                   uint32_t total_groups) {
    const uint32_t gid = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (gid >= total_groups) return;
    uint32_t lo = 0, hi = count;  // descs[lo].group_begin <= gid < descs[hi].group_begin
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) >> 1;
        if (descs[mid].group_begin <= gid) lo = mid; else hi = mid;
    }
    const PlanDesc &d = descs[lo];
    const uint32_t g = gid - d.group_begin;
    const int k = threadIdx.x & 63;
    const float xv = ((gptr_cf32)d.x)[static_cast<size_t>(g) * kGroup + k];
    const bool bad = __any(!isfinite(xv));
    float m = isfinite(xv) ? fabsf(xv) : 0.0f;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    int e = 0;
    if (m > 0.0f) (void)frexpf(m, &e);
    if (e < -100) e = -100;
    const int A = isfinite(xv) ? static_cast<int>(rintf(ldexpf(xv, 22 - e))) : 0;
    const int a0 = ((A + 128) & 255) - 128;
    const int A1 = (A - a0) >> 8;
    const int a1 = ((A1 + 128) & 255) - 128;
    const int a2 = (A1 - a1) >> 8;
    int kslot;
    const int idx = operand_index(k, kslot);
    gptr_u8 out = (gptr_u8)(d.prep + static_cast<size_t>(g) * kPrepBytes);
    out[(kslot * 4 + 0) * 16 + idx] = static_cast<uint8_t>(a0);
    out[(kslot * 4 + 1) * 16 + idx] = static_cast<uint8_t>(a1);
    out[(kslot * 4 + 2) * 16 + idx] = static_cast<uint8_t>(a2);
    out[(kslot * 4 + 3) * 16 + idx] = 0;
    if (k < 16) {
        const float f = bad ? __builtin_nanf("") : ldexpf(1.0f, e - 26);
        const uint32_t bits = __float_as_uint(f);
        out[256 + k] = k < 4 ? static_cast<uint8_t>(bits >> (8 * k)) : 0;
    }
}

// 4x4 byte transpose: d[c] holds k-pair c for rows 0..3 (one byte each);
// t[r] returns row r's k-pairs 0..3.  v_perm_b32 picks bytes of {S0:S1}
// (selector 0..3 = S1 bytes, 4..7 = S0 bytes).
__device__ __forceinline__ void transpose4(const uint32_t d0, const uint32_t d1, const uint32_t d2,
                                           const uint32_t d3, uint32_t &t0, uint32_t &t1, uint32_t &t2,
                                           uint32_t &t3) {
    const uint32_t u0 = __builtin_amdgcn_perm(d1, d0, 0x05010400u);  // (c0 r0, c1 r0, c0 r1, c1 r1)
    const uint32_t u1 = __builtin_amdgcn_perm(d1, d0, 0x07030602u);  // (c0 r2, c1 r2, c0 r3, c1 r3)
    const uint32_t u2 = __builtin_amdgcn_perm(d3, d2, 0x05010400u);  // (c2 r0, c3 r0, c2 r1, c3 r1)
    const uint32_t u3 = __builtin_amdgcn_perm(d3, d2, 0x07030602u);  // (c2 r2, c3 r2, c2 r3, c3 r3)
    t0 = __builtin_amdgcn_perm(u2, u0, 0x05040100u);
    t1 = __builtin_amdgcn_perm(u2, u0, 0x07060302u);
    t2 = __builtin_amdgcn_perm(u3, u1, 0x05040100u);
    t3 = __builtin_amdgcn_perm(u3, u1, 0x07060302u);
}

__device__ __forceinline__ uint32_t low_nibbles_x16(uint32_t t) { return (t << 4) & 0xf0f0f0f0u; }
__device__ __forceinline__ uint32_t high_nibbles_x16(uint32_t t) { return t & 0xf0f0f0f0u; }

struct StepRegs {
    uint32_t d[8];
    u32x2 s;
    i32x4 a;  // activation digits (operand A) of the group
    float f;  // group factor 2^(E-26)
};

// Code dwords and scales of one group for this lane (see the layout above).
__device__ __forceinline__ StepRegs load_step(const uint8_t *__restrict__ tile, int kslot, int q) {
    StepRegs r;
    const uint8_t *codes = tile + 64 + 32 * kslot + 4 * q;
#pragma unroll
    for (int c = 0; c < 8; ++c) r.d[c] = __builtin_nontemporal_load((gptr_u32)(codes + 128 * c));
    r.s = __builtin_nontemporal_load((gptr_u32x2)(tile + 8 * q));
    return r;
}

// acc[m] += scale(row 4j+m) * f * (D0 + 256 D1 + 65536 D2) for the four
// MFMAs of one step (meaningful in lanes 0..15).  D0 + 256*D1 is exact in
// int32 (|D| <= 2^20); the 65536*D2 term joins in fp32.
__device__ __forceinline__ void step_mfma(const StepRegs &r, const i32x4 a, const float f, float (&acc)[4]) {
    uint32_t t[8];
    transpose4(r.d[0], r.d[1], r.d[2], r.d[3], t[0], t[1], t[2], t[3]);
    transpose4(r.d[4], r.d[5], r.d[6], r.d[7], t[4], t[5], t[6], t[7]);
    const i32x4 zero = {0, 0, 0, 0};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        i32x4 b;
        b[0] = static_cast<int>(low_nibbles_x16(t[m]));
        b[1] = static_cast<int>(high_nibbles_x16(t[m]));
        b[2] = static_cast<int>(low_nibbles_x16(t[4 + m]));
        b[3] = static_cast<int>(high_nibbles_x16(t[4 + m]));
        const i32x4 dm = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, zero, 0, 0, 0);
        const int d01 = dm[0] + (dm[1] << 8);
        const float v = fmaf(static_cast<float>(dm[2]), 65536.0f, static_cast<float>(d01));
        const uint32_t sbits = (m < 2) ? r.s.x : r.s.y;
        const float sf = half_bits_to_float((m & 1) ? (sbits >> 16) : sbits) * f;
        acc[m] = fmaf(sf, v, acc[m]);
    }
}

struct Shared {
    float red[2][kWaves][kBlockRows];
    uint32_t next_item[2];
    uint32_t last;
};

// Partial sums of a 64-row block over groups [g_begin, g_end): wave w takes
// groups g_begin + w, + 4, ...; threads 0..63 return rows 0..63 of the block.
template <bool GATE>
__device__ __forceinline__ void block_partial(Shared &sh, const PlanDesc &d, uint32_t block, uint32_t g_begin,
                                              uint32_t g_end, float &out, float &gout) {
    const uint32_t groups = d.cols / kGroup;
    const uint32_t tiles = d.rows / kTileRows;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int kslot = lane >> 4, j = lane & 15, q = j & 7;
    // The second tile of a block past the last row tile re-reads the first
    // (its rows are never written).
    uint32_t tile = 2 * block + (j >> 3);
    if (tile >= tiles) tile = tiles - 1;
    const uint8_t *wt = d.w + static_cast<size_t>(tile) * groups * kTileBytes;
    const uint8_t *gt = GATE ? d.gate + static_cast<size_t>(tile) * groups * kTileBytes : nullptr;
    const uint8_t *prep = d.prep;
    float acc[4] = {0.f, 0.f, 0.f, 0.f}, gacc[4] = {0.f, 0.f, 0.f, 0.f};

    // Two register sets alternate (no copies): while one group is converted
    // and multiplied, the next group's loads are in flight.
    // The activation digits and group factor travel with the weights, one
    // step ahead of their use.
    // sched_barrier keeps the scheduler from sinking a prefetch below the
    // conversion of the previous group (which would expose its latency).
    auto load = [&](uint32_t g, StepRegs &r, StepRegs &gr) {
        r = load_step(wt + static_cast<size_t>(g) * kTileBytes, kslot, q);
        if constexpr (GATE) gr = load_step(gt + static_cast<size_t>(g) * kTileBytes, kslot, q);
        const uint8_t *pg = prep + static_cast<size_t>(g) * kPrepBytes;
        r.a = *(gptr_i32x4)(pg + 16 * (4 * kslot + (j & 3)));
        r.f = *(gptr_cf32)(pg + 256);
        __builtin_amdgcn_sched_barrier(0);
    };
    auto compute = [&](const StepRegs &r, const StepRegs &gr) {
        step_mfma(r, r.a, r.f, acc);
        if constexpr (GATE) step_mfma(gr, r.a, r.f, gacc);
    };
    // A full chunk (16 groups per wave) runs as straight-line code: the
    // waitcnt pass then counts outstanding loads exactly and each step waits
    // only for its own group while the next one is in flight.  In a runtime
    // loop it cannot track the loop-carried loads and waits for all of them
    // (vmcnt(0)), prefetch included.
    const uint32_t first = g_begin + wave;
    if (g_end - g_begin == kChunkGroups) {
        constexpr int kSteps = kChunkGroups / kWaves;
        StepRegs r[2], gr[2];
        load(first, r[0], gr[0]);
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            if (s + 1 < kSteps) load(first + (s + 1) * kWaves, r[(s + 1) & 1], gr[(s + 1) & 1]);
            compute(r[s & 1], gr[s & 1]);
        }
    } else {
        for (uint32_t g = first; g < g_end; g += kWaves) {
            StepRegs r, gr;
            load(g, r, gr);
            compute(r, gr);
        }
    }
    if (lane < 16) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            sh.red[0][wave][4 * j + m] = acc[m];
            if constexpr (GATE) sh.red[1][wave][4 * j + m] = gacc[m];
        }
    }
    __syncthreads();
    if (threadIdx.x < kBlockRows) {
        const int t = threadIdx.x;
        out = ((sh.red[0][0][t] + sh.red[0][1][t]) + sh.red[0][2][t]) + sh.red[0][3][t];
        if constexpr (GATE) gout = ((sh.red[1][0][t] + sh.red[1][1][t]) + sh.red[1][2][t]) + sh.red[1][3][t];
    }
}

template <bool GATE>
__device__ __forceinline__ void run_item(Shared &sh, const PlanDesc &d, uint32_t local) {
    const uint32_t groups = d.cols / kGroup;
    const uint32_t block = local / d.chunks, chunk = local % d.chunks;
    const uint32_t g_begin = chunk * kChunkGroups;
    const uint32_t g_end = min(groups, g_begin + kChunkGroups);
    float v = 0.f, gv = 0.f;
    block_partial<GATE>(sh, d, block, g_begin, g_end, v, gv);
    const uint32_t row = block * kBlockRows + threadIdx.x;
    const bool mine = threadIdx.x < kBlockRows && row < d.rows;
    if (d.chunks > 1) {
        // Publish this chunk; the last of the block's chunks to arrive sums
        // them in chunk order (device-scope stores, waited on before the
        // arrival count, so the summing workgroup sees them).
        if (mine) {
            store_agent(&d.partial[static_cast<size_t>(chunk) * d.rows + row], v);
            if constexpr (GATE) store_agent(&d.partial[static_cast<size_t>(d.chunks + chunk) * d.rows + row], gv);
        }
        wait_stores();
        __syncthreads();
        if (threadIdx.x == 0) sh.last = (add_agent(&d.counters[block], 1u) == d.chunks - 1) ? 1u : 0u;
        __syncthreads();
        if (sh.last == 0u) return;
        if (mine) {
            v = load_agent(&d.partial[row]);
            if constexpr (GATE) gv = load_agent(&d.partial[static_cast<size_t>(d.chunks) * d.rows + row]);
            for (uint32_t c = 1; c < d.chunks; ++c) {
                v += load_agent(&d.partial[static_cast<size_t>(c) * d.rows + row]);
                if constexpr (GATE) gv += load_agent(&d.partial[static_cast<size_t>(d.chunks + c) * d.rows + row]);
            }
        }
        if (threadIdx.x == 0) store_agent(&d.counters[block], 0u);
    }
    if (mine) {
        if (d.add != nullptr) v += ((gptr_cf32)d.add)[row];
        if constexpr (GATE) v *= silu(gv);
        ((gptr_f32)d.y)[row] = v;
    }
}

// Persistent grid: items are taken in sweep order from sched[0]; sched[1]
// counts finished workgroups and the last one resets both.
template <bool ANY_GATE>
__global__ __launch_bounds__(256) void plan_kernel(const PlanDesc *__restrict__ descs, uint32_t items,
                                                   uint32_t *__restrict__ sched) {
    __shared__ Shared sh;
    if (threadIdx.x == 0) sh.next_item[0] = add_agent(&sched[0], 1u);
    __syncthreads();
    uint32_t item = sh.next_item[0];
    uint32_t d = 0;
    int slot = 0;
    while (item < items) {
        if (threadIdx.x == 0) sh.next_item[slot ^ 1] = add_agent(&sched[0], 1u);
        while (item >= descs[d + 1].item_begin) ++d;
        const PlanDesc &desc = descs[d];
        if (ANY_GATE && desc.gate != nullptr)
            run_item<true>(sh, desc, item - desc.item_begin);
        else
            run_item<false>(sh, desc, item - desc.item_begin);
        __syncthreads();
        slot ^= 1;
        item = sh.next_item[slot];
    }
    if (threadIdx.x == 0 && add_agent(&sched[1], 1u) == gridDim.x - 1) {
        store_agent(&sched[0], 0u);
        store_agent(&sched[1], 0u);
    }
}

}  // namespace

hipError_t launch_prep(const PlanDesc *descs, uint32_t count, uint32_t groups, hipStream_t stream) {
    if (groups == 0) return hipSuccess;
    hipLaunchKernelGGL(prep_kernel, dim3((groups + 3) / 4), dim3(256), 0, stream, descs, count, groups);
    return hipGetLastError();
}

hipError_t launch_plan(const PlanDesc *descs, uint32_t items, bool any_gate, uint32_t workgroups, uint32_t *sched,
                       hipStream_t stream) {
    if (any_gate)
        hipLaunchKernelGGL(plan_kernel<true>, dim3(workgroups), dim3(256), 0, stream, descs, items, sched);
    else
        hipLaunchKernelGGL(plan_kernel<false>, dim3(workgroups), dim3(256), 0, stream, descs, items, sched);
    return hipGetLastError();
}

uint32_t plan_workgroups_per_cu(bool any_gate) { return any_gate ? 2 : 2; }

}  // namespace q4rdna
