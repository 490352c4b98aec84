// Device helpers shared by the gfx950 kernels (q4rdna_kernels.hip,
// q4rdna_mfma.hip).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "q4rdna_internal.h"

namespace q4rdna {

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Global-address-space views.  Pointers read from a descriptor table are
// generic; without the cast their loads become flat loads, which also count
// against lgkmcnt, so every wait for an LDS read would drain the in-flight
// weight loads as well.
typedef __attribute__((address_space(1))) const unsigned int *gptr_u32;
typedef __attribute__((address_space(1))) const u32x2 *gptr_u32x2;
typedef __attribute__((address_space(1))) const i32x4 *gptr_i32x4;
typedef __attribute__((address_space(1))) const f32x2 *gptr_f32x2;
typedef __attribute__((address_space(1))) const f32x4 *gptr_f32x4;
typedef __attribute__((address_space(1))) const float *gptr_cf32;
typedef __attribute__((address_space(1))) float *gptr_f32;
typedef __attribute__((address_space(1))) uint8_t *gptr_u8;
typedef __attribute__((address_space(1))) i32x4 *gptr_wi32x4;

__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
    return __half2float(__ushort_as_half(static_cast<unsigned short>(bits & 0xffffu)));
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// Cross-lane sums, v + v of lane ^ m, without LDS: m = 8 is a DPP row rotate
// by 8 (lane i of a 16-lane row reads lane (i + 8) mod 16 = i ^ 8), fused
// into the add; m = 16 and m = 32 swap rows (v_permlane16_swap) or halves
// (v_permlane32_swap) between two copies of v, after which the two copies
// hold, lane by lane, v and its partner.  fp32 addition is commutative, so
// each lane's sum equals v + partner bit for bit.
__device__ __forceinline__ float add_xor8(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false));
}
__device__ __forceinline__ float add_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// Sum over the lanes that share lane & 7 (xor 8, 16, 32, in that order).
__device__ __forceinline__ float add_over_a(float v) { return add_xor32(add_xor16(add_xor8(v))); }

// add_over_a of four values at once, the result transposed: lane l returns
// the sum of v[l >> 4] (over the lanes sharing l & 7).  The row swaps pair
// v[0] with v[1] and v[2] with v[3], so each permlane swap and add reduces
// two of the values; every lane-row's sum has add_over_a's operands in
// add_over_a's order, so the sums are the same bits.
__device__ __forceinline__ float add_over_a4(const float (&v)[4]) {
    const float v0 = add_xor8(v[0]), v1 = add_xor8(v[1]), v2 = add_xor8(v[2]), v3 = add_xor8(v[3]);
    // Lane-rows 0..3 of s01: v0 (rows 0+1), v1 (rows 0+1), v0 (rows 2+3), v1 (rows 2+3).
    const auto p01 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v0), __float_as_uint(v1), false, false);
    const float s01 = __uint_as_float(p01[0]) + __uint_as_float(p01[1]);
    const auto p23 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v2), __float_as_uint(v3), false, false);
    const float s23 = __uint_as_float(p23[0]) + __uint_as_float(p23[1]);
    // Lanes 0..31 take s01's halves, lanes 32..63 s23's.
    const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(s01), __float_as_uint(s23), false, false);
    return __uint_as_float(h[0]) + __uint_as_float(h[1]);
}

// n / d for d = split, n * d < 2^32: magic = ceil(2^32 / d) for d > 1
// (split_magic on the host), 0 for d = 1.
__device__ __forceinline__ uint32_t div_split(uint32_t n, uint32_t d, uint32_t magic) {
    return d == 1 ? n : __umulhi(n, magic);
}

// The wave's index in its workgroup, as a wave-uniform (scalar) value, so
// that addresses built from it stay in scalar registers.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6)); }

// Device-scope (agent) relaxed atomics: on gfx950 these are single sc1
// loads/stores and a plain atomic add, coherent across the XCDs' L2s without
// the whole-L2 write-back/invalidate that release/acquire fences emit.  Every
// pointer passed here is device memory; the global address space keeps them
// global_* instructions: a flat access also counts against lgkmcnt, so the
// next wait for an LDS read would wait for the store's acknowledgement too.
typedef __attribute__((address_space(1))) uint32_t *gptr_au32;
__device__ __forceinline__ void store_agent(float *p, float v) {
    __hip_atomic_store((gptr_f32)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent(uint32_t *p, uint32_t v) {
    __hip_atomic_store((gptr_au32)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float *p) {
    return __hip_atomic_load((gptr_cf32)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t add_agent(uint32_t *p, uint32_t v) {
    return __hip_atomic_fetch_add((gptr_au32)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until this wave's stores have completed (visible at device scope for
// sc1 stores); the memory clobber keeps the compiler from moving memory
// operations across it.
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Two K chunks of a row meet in one exchange slot (zero between launches):
// each chunk's workgroup swaps its partial sums, XOR kSlotKey, into the slot
// with one device-scope atomic.  The first to arrive reads zero back and is
// done; the second reads the first's partials, adds its own -- fp32 addition
// is commutative, so the sum is the same whichever chunk came first -- and
// puts zero back.  One atomic round trip replaces a partial store, its
// acknowledgement, an arrival count and a reload of the partials.  A partial
// whose bits equal kSlotKey (a signaling NaN, which arithmetic never
// produces) would store as zero, so it is sent as a quiet NaN.  GATE: the
// slot is the 64-bit pair (sum, SwiGLU gate sum) at words 2*row, 2*row + 1,
// and only the sum's word tells an empty slot; otherwise word row.  Both
// layouts keep every word zero between launches, so one slot region serves
// both, and zero-filled memory is a valid empty region.
typedef __attribute__((address_space(1))) uint64_t *gptr_au64;
__device__ __forceinline__ uint32_t slot_word(float v) {
    const uint32_t b = __float_as_uint(v);
    return (b == kSlotKey ? kSlotQuietNan : b) ^ kSlotKey;
}
template <bool GATE>
__device__ __forceinline__ bool exchange_pair(uint32_t *slots, uint32_t row, float &v, float &gv) {
    if constexpr (GATE) {
        gptr_au64 p = (gptr_au64)slots + row;
        const uint64_t mine = (static_cast<uint64_t>(__float_as_uint(gv) ^ kSlotKey) << 32) | slot_word(v);
        const uint64_t got = __hip_atomic_exchange(p, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (static_cast<uint32_t>(got) == 0u) return false;
        v = __uint_as_float(static_cast<uint32_t>(got) ^ kSlotKey) + v;
        gv = __uint_as_float(static_cast<uint32_t>(got >> 32) ^ kSlotKey) + gv;
        __hip_atomic_store(p, uint64_t{0}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        gptr_au32 p = (gptr_au32)slots + row;
        const uint32_t got = __hip_atomic_exchange(p, slot_word(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (got == 0u) return false;
        v = __uint_as_float(got ^ kSlotKey) + v;
        __hip_atomic_store(p, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return true;
}

// Chunk s of `split` K chunks (split >= 2) meets the others in a fixed binary
// tree of exchange slots.  With P the smallest power of two >= split, chunk s
// is leaf P + s of a heap and internal node k (1 <= k < P) owns slot region
// k - 1: `rows` slots, two words per row with a gate.  Going up, each node
// whose other subtree holds a chunk takes one exchange_pair; a node whose
// right subtree lies past the last chunk is passed straight through.  The
// first arrival at a node stops there, the second carries both subtrees' sum
// up, and the thread that clears the root holds the row's whole sum (returns
// true).  A node's two inputs are fixed sums and fp32 addition is
// commutative, so the root sum -- ((p0 + p1) + (p2 + p3)) + (p4 + p5) at
// split 6 -- is the same whichever chunk arrives first; at split 2 the tree
// is the single exchange.  Every slot a launch uses is swapped into exactly
// twice, so all are zero again when it ends.
template <bool GATE>
__device__ __forceinline__ bool exchange_tree(uint32_t *slots, uint32_t rows, uint32_t split, uint32_t s,
                                              uint32_t row, float &v, float &gv) {
    const uint32_t P = 1u << (32 - __builtin_clz(split - 1u));  // exchange_leaves(split)
    uint32_t node = P + s;
    for (uint32_t d = 0; node > 1u; ++d, node >>= 1) {
        if (exchange_meets(node, d, P, split)) {
            uint32_t *region = slots + static_cast<size_t>((node >> 1) - 1u) * rows * (GATE ? 2u : 1u);
            if (!exchange_pair<GATE>(region, row, v, gv)) return false;
        }
    }
    return true;
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// A lane's tile slice: dword j of the 1,024 code bytes at 32 * (a + 8j) +
// 4q holds rows 4q..4q+3 at k-pair a + 8j (a = lane >> 3, q = lane & 7 in
// the kernels that read it).  Its 32 codes as fp16 subnormals: for k-pair
// a + 8j, l02[j] = (u of row 4q, u of row 4q+2) at even k, h02[j] = 16u of
// the same rows at odd k, l13/h13 the same for rows 4q+1 and 4q+3.
struct TileCodes {
    f16x2 l02[4], h02[4], l13[4], h13[4];
};

__device__ __forceinline__ TileCodes split_codes(const uint32_t (&dw)[4]) {
    TileCodes w;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        // (d & mask) ^ offset is one v_bitop3_b32 each.
        const uint32_t d = dw[j], o = d >> 8;
        w.l02[j] = __builtin_bit_cast(f16x2, (d & 0x000f000fu) ^ 0x00080008u);
        w.h02[j] = __builtin_bit_cast(f16x2, (d & 0x00f000f0u) ^ 0x00800080u);
        w.l13[j] = __builtin_bit_cast(f16x2, (o & 0x000f000fu) ^ 0x00080008u);
        w.h13[j] = __builtin_bit_cast(f16x2, (o & 0x00f000f0u) ^ 0x00800080u);
    }
    return w;
}

// acc[r] += scale(row 4q + r) * (c + sum over the lane's 8 k of u * x), the
// row's products in k order: for each k-pair the even k, then the odd k.
// xl = even-k x * 2^24, xh = odd-k x * 2^20.
__device__ __forceinline__ void apply_codes(const TileCodes &w, uint32_t s01, uint32_t s23, const float4 xl,
                                            const float4 xh, const float c, float (&acc)[4]) {
    const float xlv[4] = {xl.x, xl.y, xl.z, xl.w};
    const float xhv[4] = {xh.x, xh.y, xh.z, xh.w};
    float p0 = c, p1 = c, p2 = c, p3 = c;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        p0 = fmaf(static_cast<float>(w.l02[j].x), xlv[j], p0);
        p1 = fmaf(static_cast<float>(w.l13[j].x), xlv[j], p1);
        p2 = fmaf(static_cast<float>(w.l02[j].y), xlv[j], p2);
        p3 = fmaf(static_cast<float>(w.l13[j].y), xlv[j], p3);
        p0 = fmaf(static_cast<float>(w.h02[j].x), xhv[j], p0);
        p1 = fmaf(static_cast<float>(w.h13[j].x), xhv[j], p1);
        p2 = fmaf(static_cast<float>(w.h02[j].y), xhv[j], p2);
        p3 = fmaf(static_cast<float>(w.h13[j].y), xhv[j], p3);
    }
    acc[0] = fmaf(half_bits_to_float(s01), p0, acc[0]);
    acc[1] = fmaf(half_bits_to_float(s01 >> 16), p1, acc[1]);
    acc[2] = fmaf(half_bits_to_float(s23), p2, acc[2]);
    acc[3] = fmaf(half_bits_to_float(s23 >> 16), p3, acc[3]);
}

// Activation factors for apply_codes: x * 2^24 at even k, x * 2^20 at odd
// k (the 1/16 of the high nibbles folded in); every product is then exactly
// u * x.  The staged values are finite for |x| < 2^104.
constexpr float kEvenScale = 16777216.0f;  // 2^24
constexpr float kOddScale = 1048576.0f;    // 2^20 = 2^24 / 16

// Workgroups are dealt to the 8 XCDs round robin; remap so consecutive
// logical indices run on one XCD.  A bijection on [0, n).
__device__ __forceinline__ uint32_t xcd_remap(uint32_t b, uint32_t n) {
    const uint32_t xcd = b & 7u, idx = b >> 3, per = n >> 3, rem = n & 7u;
    return xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
}

}  // namespace q4rdna
