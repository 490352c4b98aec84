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
//  * v_mfma_i32_16x16x64_i8: D[i][j] = sum_k A[i][k] B[k][j] with A = digit
//    rows of x and B = 16 weight rows, one group (64 k) per instruction;
//    |D| <= 64 * 128 * 128 = 2^20, exact in int32.  Lane l supplies 16 bytes
//    of A row l%16 and of B column l%16 for k-slot l/16 and receives
//    D[4*(l/16) + v][l%16] in element v -- checked on the device against a
//    CPU product.  Per (row, group) the result is
//    scale * 2^(E-26) * (D0 + 256*D1 + 65536*D2) (2^-4 undoes the 16*q).
//
//  * Operand order.  A lane's 16 operand bytes for k-slot kslot are, for
//    e = 0..15, k = 2*(16*(e/8) + 4*(e%4) + kslot) + (e/4)%2 within the group:
//    the low and high nibbles of k-pairs kslot + 4c, c = 0..7, which is what
//    a 4x4 byte transpose (v_perm_b32) of four code dwords -- four rows at
//    one k-pair each -- followed by the nibble split produces.  The
//    activation digits are stored in the same order.
//
// The sweep kernel's lane mapping is described at the kernel below.
#include "q4rdna_device.h"

namespace q4rdna {
namespace {

constexpr int kWaves = 4;

// Activation digits.  One lane takes one k-slot of a 64-element group: the
// 16 elements 2*(kslot + 4c) + h (c = 0..7, h = 0..1), i.e. its operand bytes
// e = 8*(c/4) + 4*h + c%4.  The group's block exponent E (frexp of max |x|)
// and non-finite flag are reduced over the four lanes holding its k-slots
// (lanes 4p .. 4p+3 of the wave); each element becomes A = rint(x*2^(22-E)),
// split into three balanced int8 digits.  A lane's three digit rows are 48
// contiguous bytes (row d at 16*d) of a 64-byte k-slot record: the
// single-vector and batched layouts both keep a k-slot's rows together.  Row
// 3 feeds MFMA rows that are discarded; it is written as zeros where the
// record is written whole (prep_kslot's `pad`).  `have` false:
// the lane's group lies past the end: it loads a readable stand-in group,
// discards the values and writes nothing; its three sibling lanes are in
// the same state.

// The lane's 16 elements in operand order; x 8-byte aligned and readable
// even where `have` is false (its values are then replaced by zeros).  The
// eight loads are unconditional so that they issue back to back: guarded
// loads make the compiler wait for each pair inside its branch, four
// dependent round trips to memory.
__device__ __forceinline__ void load_kslot(const float *x, int kslot, bool have, float (&xs)[16]) {
    f32x2 v[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) v[c] = *(gptr_f32x2)(x + 2 * (kslot + 4 * c));
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        xs[8 * (c >> 2) + (c & 3)] = have ? v[c][0] : 0.0f;
        xs[8 * (c >> 2) + 4 + (c & 3)] = have ? v[c][1] : 0.0f;
    }
}

// The same for x that is only 4-byte aligned (the per-tensor entry points'
// contract), without branches: x must point at a readable group even where
// `have` is false (its values are then replaced by zeros), so that the
// loads issue back to back and nothing waits for one before the next
// (a guarded load makes the compiler wait for it inside its branch).
// Cached loads: every unit of a launch reads the same x.
__device__ __forceinline__ void load_kslot_f32_always(const float *x, int kslot, bool have, float (&xs)[16]) {
    float v[16];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        v[2 * c] = *(gptr_cf32)(x + 2 * (kslot + 4 * c));
        v[2 * c + 1] = *(gptr_cf32)(x + 2 * (kslot + 4 * c) + 1);
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        xs[8 * (c >> 2) + (c & 3)] = have ? v[2 * c] : 0.0f;
        xs[8 * (c >> 2) + 4 + (c & 3)] = have ? v[2 * c + 1] : 0.0f;
    }
}

// Digits of the lane's elements (rows[d] = digit d of the 16 elements) and
// the group's exponent and non-finite flag.  Every lane of the wave runs the
// shuffles; rows are only meaningful where `have`.
__device__ __forceinline__ void kslot_digits(const float (&xs)[16], bool have, i32x4 (&rows)[3], bool &bad,
                                             int &e_out) {
    float m = 0.0f;
    bool nonfinite = false;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        nonfinite |= !isfinite(xs[i]);
        m = fmaxf(m, isfinite(xs[i]) ? fabsf(xs[i]) : 0.0f);
    }
    // The group's four lanes are a DPP quad: xor 1 and xor 2 as quad
    // permutes ([1,0,3,2] and [2,3,0,1]), no LDS round trip.
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), 0xB1, 0xf, 0xf, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), 0x4E, 0xf, 0xf, false)));
    int nf = nonfinite ? 1 : 0;
    nf |= __builtin_amdgcn_mov_dpp(nf, 0xB1, 0xf, 0xf, false);
    nf |= __builtin_amdgcn_mov_dpp(nf, 0x4E, 0xf, 0xf, false);
    int e = 0;
    if (m > 0.0f) (void)frexpf(m, &e);
    if (e < -100) e = -100;
    bad = nf != 0;
    e_out = e;
    uint32_t row[3][4] = {};
    if (have) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int A = isfinite(xs[i]) ? static_cast<int>(rintf(ldexpf(xs[i], 22 - e))) : 0;
            const int a0 = ((A + 128) & 255) - 128;
            const int A1 = (A - a0) >> 8;
            const int a1 = ((A1 + 128) & 255) - 128;
            const int a2 = (A1 - a1) >> 8;
            const int sh = 8 * (i & 3);
            row[0][i >> 2] |= (static_cast<uint32_t>(a0) & 255u) << sh;
            row[1][i >> 2] |= (static_cast<uint32_t>(a1) & 255u) << sh;
            row[2][i >> 2] |= (static_cast<uint32_t>(a2) & 255u) << sh;
        }
    }
#pragma unroll
    for (int d = 0; d < 3; ++d)
        rows[d] = i32x4{static_cast<int>(row[d][0]), static_cast<int>(row[d][1]), static_cast<int>(row[d][2]),
                        static_cast<int>(row[d][3])};
}

// Group factor 2^(E-26) of the digits (NaN for a non-finite group).
__device__ __forceinline__ float digit_factor(bool bad, int e) { return bad ? __builtin_nanf("") : ldexpf(1.0f, e - 26); }

// With `pad` the k-slot's record is written whole, row 3 as zeros (stores
// that cover whole 64-byte runs measured 0.7 us faster over a 20,736-group
// stack than leaving a 16-byte hole in every record).  The stores are
// nontemporal: the digits then leave the L2 as they are written instead of
// at the end of the launch, and the sweep launch after it started 2.2 us
// sooner.
__device__ __forceinline__ void prep_kslot(const float *x, int kslot, bool have, bool pad, gptr_u8 out, bool &bad,
                                           int &e_out) {
    float xs[16];
    load_kslot(x, kslot, have, xs);
    i32x4 rows[3];
    kslot_digits(xs, have, rows, bad, e_out);
    if (!have) return;
#pragma unroll
    for (int d = 0; d < 3; ++d) __builtin_nontemporal_store(rows[d], (gptr_wi32x4)(out + 16 * d));
    if (pad) __builtin_nontemporal_store(i32x4{0, 0, 0, 0}, (gptr_wi32x4)(out + 48));
}

// Single-vector layout per group (kPrepBytes = 272): byte (kslot*4 + d)*16 + e
// for digit d (row d = 3 holds zeros), the float factor 2^(E-26) at 256 (NaN
// for a non-finite group) followed by 12 zero bytes.  Lane 4p + kslot of a
// wave converts k-slot kslot of the wave's group p (16 groups per wave);
// group_x[g] is the address of global group g's 64 activations (built by the
// host); its digits go to prep + g * kPrepBytes.
__global__ __launch_bounds__(256) void prep_kernel(const float *const *__restrict__ group_x,
                                                   uint8_t *__restrict__ prep, uint32_t total_groups) {
    const int lane = threadIdx.x & 63, kslot = lane & 3;
    const uint32_t gid = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 16 + (lane >> 2);
    const bool valid = gid < total_groups;
    const float *x = group_x[valid ? gid : total_groups - 1];
    gptr_u8 out = (gptr_u8)(prep + static_cast<size_t>(valid ? gid : 0) * kPrepBytes);
    bool bad;
    int e;
    prep_kslot(x, kslot, valid, true, out + 64 * kslot, bad, e);
    if (valid && kslot == 0)
        __builtin_nontemporal_store(i32x4{static_cast<int>(__float_as_uint(digit_factor(bad, e))), 0, 0, 0},
                                    (gptr_wi32x4)(out + 256));
}

// The VALU sweep's prepare (kSweepValu): per group (kPrepBytes = 288), for
// lane slot a = 0..7 (k-pairs a + 8j, j = 0..3) the float4 of its even-k
// x * 2^24 at 16a, the float4 of its odd-k x * 2^20 at 128 + 16a and
// c = -8 * the sum of its eight x at 256 + 4a: what the per-tensor kernels
// stage in LDS, in the same order of additions.  One thread per (group,
// slot); nontemporal stores, as the digit prepare's.
__global__ __launch_bounds__(256) void prep_valu_kernel(const float *const *__restrict__ group_x,
                                                        uint8_t *__restrict__ prep, uint32_t groups) {
    const uint32_t item = blockIdx.x * 256u + threadIdx.x;
    if (item >= groups * 8u) return;
    const uint32_t g = item >> 3, a = item & 7u;
    const gptr_cf32 x = (gptr_cf32)group_x[g] + 2 * a;
    float l[4], h[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        l[j] = x[16 * j];
        h[j] = x[16 * j + 1];
    }
    gptr_u8 out = (gptr_u8)(prep + static_cast<size_t>(g) * kPrepBytes);
    const f32x4 xl = {l[0] * kEvenScale, l[1] * kEvenScale, l[2] * kEvenScale, l[3] * kEvenScale};
    const f32x4 xh = {h[0] * kOddScale, h[1] * kOddScale, h[2] * kOddScale, h[3] * kOddScale};
    __builtin_nontemporal_store(xl, (__attribute__((address_space(1))) f32x4 *)(out + 16 * a));
    __builtin_nontemporal_store(xh, (__attribute__((address_space(1))) f32x4 *)(out + 128 + 16 * a));
    const float c = -8.0f * (((((((l[0] + h[0]) + l[1]) + h[1]) + l[2]) + h[2]) + l[3]) + h[3]);
    __builtin_nontemporal_store(c, (gptr_f32)(out + 256 + 4 * a));
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

// ---- sweep kernel ---------------------------------------------------------
//
// An item is (64-row block, stream, K chunk of up to kChunkGroups = 192
// groups), taken by one workgroup.  Its four waves read the block's two row
// tiles side by side: in workgroup step s, wave w takes groups
// g0 + 4w .. g0 + 4w + 3 with g0 = chunk start + 16s, so the workgroup
// streams two contiguous runs of 16 tiles.  A 192-group chunk holds a whole
// 12288-wide row, so such GEMVs finish without split-K partials: an item's
// end (a workgroup barrier, the reduction, and for split items an arrival
// chain through global memory) is where the sweep stalls.
//
// Loads.  Per step a wave reads eight tiles (4 groups x 2 row tiles).  Load
// instruction c reads the whole 1024-byte code area of tile (group c/2, row
// tile c%2), 16 contiguous bytes per lane -- long contiguous runs per
// instruction stream markedly faster than short ones -- straight into the
// wave's LDS stage (global_load_lds_dwordx4), where each lane then picks up
// its operand bytes.  (A short tail loads into registers and restages.)
// The LDS copy of tile c starts at kStageStride*c; the skew past 1024 bytes
// spreads the operand reads of the eight copies over the LDS banks.
//
// Operands.  Lane l = 16*kslot + j with j = 4*gB + r4 and r4 = 2*T + h:
//  * B: from the copy of tile (gB, T) the lane reads rows 16h..16h+15 at
//    k-pairs kslot + 4c, c = 0..7 (eight 16-byte LDS reads).  Dword m of read
//    c holds rows 16h + 4m..+3 of k-pair kslot + 4c, so the 4x4 transposes
//    above give, for row n = 4m + q, the operand of MFMA n (16 MFMAs per
//    step, one per row).
//  * A: digit (j & 3) of group g0 + 4w + gB at k-slot kslot, so rows
//    4s'..4s'+3 of A hold group g0 + 4w + s'.
//  * D: lane l holds D rows 4*(l/16)..+3 of column j: group kslot's digits
//    times column j's rows of group gB.  Meaningful when gB == kslot -- lanes
//    20*gB + r4, which accumulate rows 32T + 16h + n, with the fp16 scales of
//    those rows loaded by the same lane; the 16 (wave, gB) partial sums of
//    each row meet in LDS at the item's end.
constexpr int kStepGroups = 4;                         // groups per wave step
constexpr int kWgStepGroups = kWaves * kStepGroups;    // groups per workgroup step
static_assert(kChunkGroups % kWgStepGroups == 0, "chunks are whole workgroup steps");
// LDS bytes per staged tile: 1024 + a 64-byte skew.  Over the 252-tensor
// stack the 64-byte skew measures 10.2M SQ_LDS_BANK_CONFLICT cycles against
// 23.7M for a 32- or 128-byte skew and 50.9M for none, at equal sweep time.
constexpr int kStageStride = 1088;
constexpr int kStageBytes = 8 * kStageStride;          // per wave

struct WaveRegs {
    i32x4 code[8];  // the operand bytes read from the LDS stage (a short tail first holds tile c's 16 bytes at 16*lane)
    i32x4 sc[2];    // the lane's 16 rows' fp16 scales
    i32x4 a;        // activation digits
    float f;        // group factor of the lane's D rows
};

struct LaneRole {
    int kslot, gB, T, h;
    uint32_t a_offset;   // digit bytes within a prep group
    uint32_t lds_read;   // byte offset of the lane's first operand read in a staged step
    bool useful;         // gB == kslot
};

__device__ __forceinline__ LaneRole lane_role(int lane) {
    LaneRole r;
    r.kslot = lane >> 4;
    const int j = lane & 15;
    r.gB = j >> 2;
    r.T = (j >> 1) & 1;
    r.h = j & 1;
    r.a_offset = 16u * (4u * r.kslot + (j & 3));
    r.lds_read = kStageStride * (2 * r.gB + r.T) + 32 * r.kslot + 16 * r.h;
    r.useful = r.gB == r.kslot;
    return r;
}

// Through this wave's LDS stage: store the eight tiles, read the operand
// bytes back in their place.  LDS operations of one wave complete in order,
// so the reads see the stores and the next step's stores follow the reads.
__device__ __forceinline__ void restage(WaveRegs &r, uint8_t *stage, const LaneRole &ln, int lane) {
#pragma unroll
    for (int c = 0; c < 8; ++c) *reinterpret_cast<i32x4 *>(stage + kStageStride * c + 16 * lane) = r.code[c];
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int c = 0; c < 8; ++c) r.code[c] = *reinterpret_cast<const i32x4 *>(stage + ln.lds_read + 128 * c);
}

// Load a tile's 1024 code bytes straight into LDS (global_load_lds_dwordx4,
// 16 bytes per lane at dst + 16*lane; dst is wave-uniform), nontemporal so
// the weight stream does not displace cached data (without it the sweep
// measured 5 % slower).  The caller waits with wait_vm_all() before reading
// the bytes and keeps every read of dst before the next load into it.
constexpr int kLdsDmaNontemporal = 2;  // cache-policy operand: nt
__device__ __forceinline__ void code_to_lds(const uint8_t *tile, uint8_t *dst, int lane) {
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(tile + 64 + 16 * lane),
                                     (__attribute__((address_space(3))) void *)dst, 16, 0, kLdsDmaNontemporal);
}
__device__ __forceinline__ void wait_vm_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
__device__ __forceinline__ void wait_lds_all() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// acc[n] += scale(row n) * f * (D0 + 256 D1 + 65536 D2) for the 16 MFMAs of
// one step (meaningful in the useful lanes).  D0 + 256*D1 is exact in int32
// (|D| <= 2^20); the 65536*D2 term joins in fp32.  MASK: skip the update
// where the lane's D group lies past the chunk.
template <bool MASK>
__device__ __forceinline__ void compute_wave(const WaveRegs &r, float (&acc)[16], bool valid) {
    const i32x4 zero = {0, 0, 0, 0};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        uint32_t t[8];
        transpose4(r.code[0][m], r.code[1][m], r.code[2][m], r.code[3][m], t[0], t[1], t[2], t[3]);
        transpose4(r.code[4][m], r.code[5][m], r.code[6][m], r.code[7][m], t[4], t[5], t[6], t[7]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int n = 4 * m + q;
            i32x4 b;
            b[0] = static_cast<int>(low_nibbles_x16(t[q]));
            b[1] = static_cast<int>(high_nibbles_x16(t[q]));
            b[2] = static_cast<int>(low_nibbles_x16(t[4 + q]));
            b[3] = static_cast<int>(high_nibbles_x16(t[4 + q]));
            const i32x4 dm = __builtin_amdgcn_mfma_i32_16x16x64_i8(r.a, b, zero, 0, 0, 0);
            const int d01 = dm[0] + (dm[1] << 8);
            const float v = fmaf(static_cast<float>(dm[2]), 65536.0f, static_cast<float>(d01));
            const uint32_t word = static_cast<uint32_t>(r.sc[n >> 3][(n >> 1) & 3]);
            const float sf = half_bits_to_float((n & 1) ? (word >> 16) : word) * r.f;
            const float upd = fmaf(sf, v, acc[n]);
            acc[n] = (!MASK || valid) ? upd : acc[n];
        }
    }
}

// compute_wave with the 16 MFMAs issued back to back into their own
// results before any of them is used, so their latencies overlap; for
// workgroups with one wave per SIMD, where nothing else hides them.  Same
// arithmetic, same order of the fp32 updates.
template <bool MASK>
__device__ __forceinline__ void compute_wave_batched(const WaveRegs &r, float (&acc)[16], bool valid) {
    const i32x4 zero = {0, 0, 0, 0};
    i32x4 dm[16];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        uint32_t t[8];
        transpose4(r.code[0][m], r.code[1][m], r.code[2][m], r.code[3][m], t[0], t[1], t[2], t[3]);
        transpose4(r.code[4][m], r.code[5][m], r.code[6][m], r.code[7][m], t[4], t[5], t[6], t[7]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            i32x4 b;
            b[0] = static_cast<int>(low_nibbles_x16(t[q]));
            b[1] = static_cast<int>(high_nibbles_x16(t[q]));
            b[2] = static_cast<int>(low_nibbles_x16(t[4 + q]));
            b[3] = static_cast<int>(high_nibbles_x16(t[4 + q]));
            dm[4 * m + q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(r.a, b, zero, 0, 0, 0);
        }
    }
#pragma unroll
    for (int n = 0; n < 16; ++n) {
        const int d01 = dm[n][0] + (dm[n][1] << 8);
        const float v = fmaf(static_cast<float>(dm[n][2]), 65536.0f, static_cast<float>(d01));
        const uint32_t word = static_cast<uint32_t>(r.sc[n >> 3][(n >> 1) & 3]);
        const float sf = half_bits_to_float((n & 1) ? (word >> 16) : word) * r.f;
        const float upd = fmaf(sf, v, acc[n]);
        acc[n] = (!MASK || valid) ? upd : acc[n];
    }
}

// ---- the VALU formulation of a step (kSweepValu) ----------------------------
//
// The same eight tiles in the wave's LDS stage (group gB = c/2, row tile
// T = c%2 at kStageStride*c), read in the per-tensor kernels' lane layout:
// lane (q = lane & 7, a = lane >> 3) takes dwords 32*(a + 8j) + 4q, j = 0..3
// (rows 4q..4q+3 at k-pairs a + 8j; the 64 lanes of one read hit 64
// consecutive dwords), and accumulates
// acc[T][r] += scale(row 4q + r) * (c + sum of u * x) with v_fma_mix_f32
// on fp16-subnormal codes, as gemv_kernel does.  Scales (8 bytes per tile)
// and the prepared x of the step's four groups go to registers.
struct ValuAux {
    u32x2 sc[8];               // tile c: fp16 scales of rows 4q..4q+3
    f32x4 xl[4], xh[4];        // group gB: even-k x * 2^24, odd-k x * 2^20 at the lane's k-pairs
    float xc[4];               // group gB: -8 * the sum of the lane's eight x
};
struct ValuRegs {
    i32x4 code[8];  // the tiles' code bytes as loaded, 16 per lane (a step loaded across an item's end)
    ValuAux aux;
};

// Scales of tiles (group g0 + c/2 clamped to g_last, row tile c%2) and the
// prepared x of groups g0..g0+3 (clamped).
__device__ __forceinline__ void load_valu_aux(ValuAux &r, const uint8_t *rt0, const uint8_t *rt1,
                                              const uint8_t *prep, uint32_t g0, uint32_t g_last, int q, int a) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const uint32_t g = min(g0 + (c >> 1), g_last);
        r.sc[c] = __builtin_nontemporal_load(
            (gptr_u32x2)(((c & 1) ? rt1 : rt0) + static_cast<size_t>(g) * kTileBytes + 8 * q));
    }
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
        const uint8_t *px = prep + static_cast<size_t>(min(g0 + gi, g_last)) * kPrepBytes;
        r.xl[gi] = *(gptr_f32x4)(px + 16 * a);
        r.xh[gi] = *(gptr_f32x4)(px + 128 + 16 * a);
        r.xc[gi] = *(gptr_cf32)(px + 256 + 4 * a);
    }
}

// MASK: groups gi >= valid_groups of the step lie past the chunk.
template <bool MASK>
__device__ __forceinline__ void compute_valu(const uint8_t *stage, const ValuAux &r, float (&acc)[2][4], int q,
                                             int a, uint32_t valid_groups) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int gi = c >> 1, T = c & 1;
        uint32_t d[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            d[j] = *reinterpret_cast<const uint32_t *>(stage + kStageStride * c + 32 * (a + 8 * j) + 4 * q);
        float t[4] = {acc[T][0], acc[T][1], acc[T][2], acc[T][3]};
        apply_codes(split_codes(d), r.sc[c].x, r.sc[c].y, make_float4(r.xl[gi][0], r.xl[gi][1], r.xl[gi][2], r.xl[gi][3]),
                    make_float4(r.xh[gi][0], r.xh[gi][1], r.xh[gi][2], r.xh[gi][3]), r.xc[gi], t);
        if (!MASK || static_cast<uint32_t>(gi) < valid_groups) {
#pragma unroll
            for (int k = 0; k < 4; ++k) acc[T][k] = t[k];
        }
    }
}

// Where an item's 64 sums go: y directly when the block has one item, else
// part `part` of the block's per = streams * chunks parts.
struct ItemOut {
    const float *add;
    float *y;
    float *partial;
    uint32_t *counters;
    uint32_t rows, block, part, per, chunks, streams;
};

// One item's reduction buffer: [0] W, [1] the SwiGLU gate of a one-item
// block, or the two row blocks of a pair item.
using Red = float[2][kWaves][kStepGroups][kBlockRows];

// The useful lanes publish their 16 rows; thread t < 64 then sums row t's 16
// (wave, group) partials in a fixed order and finishes the item: y = sum
// (+ add), or the part is published and the block's last part to arrive sums
// the parts in chunk order (device-scope stores, drained before the arrival
// count, so the summing workgroup sees them) and applies the epilogue.
// GLU: the item streamed W into acc and the SwiGLU gate into gacc (a block
// with one item); y = (sum + add) * silu(gate sum), the arrival chain's
// epilogue without the chain.
// `last` is the workgroup's word for the arrival result.
template <bool GLU, int G>
__device__ __forceinline__ void finish_item_sum(Red &red, uint32_t &last, const ItemOut &o);

template <bool GLU>
__device__ __forceinline__ void finish_item(Red &red, uint32_t &last, const ItemOut &o, const float (&acc)[16],
                                            const float (&gacc)[16], const LaneRole &ln, int wave) {
    if (ln.useful) {
        float *dst = &red[0][wave][ln.gB][32 * ln.T + 16 * ln.h];
#pragma unroll
        for (int n = 0; n < 16; ++n) dst[n] = acc[n];
        if constexpr (GLU) {
            float *gdst = &red[1][wave][ln.gB][32 * ln.T + 16 * ln.h];
#pragma unroll
            for (int n = 0; n < 16; ++n) gdst[n] = gacc[n];
        }
    }
    finish_item_sum<GLU, kStepGroups>(red, last, o);
}

// After the publish: thread t < 64 sums row t's partials red[.][w][g][t]
// for w < kWaves, g < G in that order (G = kStepGroups for the MFMA
// formulation, whose lanes publish per group; 1 for the VALU one, whose
// lanes sum their groups themselves) and finishes the item.
template <bool GLU, int G>
__device__ __forceinline__ void finish_item_sum(Red &red, uint32_t &last, const ItemOut &o) {
    __syncthreads();
    const uint32_t row = o.block * kBlockRows + threadIdx.x;
    const bool mine = threadIdx.x < kBlockRows && row < o.rows;
    float v = 0.0f, gv = 0.0f;
    if (threadIdx.x < kBlockRows) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
#pragma unroll
            for (int g = 0; g < G; ++g) v += red[0][w][g][threadIdx.x];
        if constexpr (GLU) {
#pragma unroll
            for (int w = 0; w < kWaves; ++w)
#pragma unroll
                for (int g = 0; g < G; ++g) gv += red[1][w][g][threadIdx.x];
        }
    }
    if (o.per == 1) {
        if (mine) {
            if (o.add != nullptr) v += ((gptr_cf32)o.add)[row];
            if constexpr (GLU) v *= silu(gv);
            __builtin_nontemporal_store(v, (gptr_f32)o.y + row);
        }
        return;
    }
    if (mine) store_agent(&o.partial[static_cast<size_t>(o.part) * o.rows + row], v);
    wait_stores();
    __syncthreads();
    if (threadIdx.x == 0) last = (add_agent(&o.counters[o.block], 1u) == o.per - 1) ? 1u : 0u;
    __syncthreads();
    if (last == 0u) return;
    if (mine) {
        float u = load_agent(&o.partial[row]);
        for (uint32_t k = 1; k < o.chunks; ++k) u += load_agent(&o.partial[static_cast<size_t>(k) * o.rows + row]);
        if (o.add != nullptr) u += ((gptr_cf32)o.add)[row];
        if (o.streams > 1) {
            const float *gp = o.partial + static_cast<size_t>(o.chunks) * o.rows;
            float g = load_agent(&gp[row]);
            for (uint32_t k = 1; k < o.chunks; ++k) g += load_agent(&gp[static_cast<size_t>(k) * o.rows + row]);
            u *= silu(g);
        }
        __builtin_nontemporal_store(u, (gptr_f32)o.y + row);
    }
    if (threadIdx.x == 0) store_agent(&o.counters[o.block], 0u);
}

// The reduction buffers alternate by item parity, so an item needs one
// workgroup barrier: the next item's writes go to the other buffer, and the
// one after that's writes follow that item's barrier, which the waves still
// summing this item reach only once they are done.
struct Shared {
    uint8_t stage[kWaves][kStageBytes];
    Red red[2];
    uint32_t last;
};

// The end of a pair item (two 64-row blocks, 128 rows from row
// 128 * o.block): acc0 / acc1 hold the blocks' sums in the useful lanes;
// thread t < 128 sums row t's 16 (wave, group) partials in the fixed order
// and writes y (+ add).
template <int G>
__device__ __forceinline__ void finish_pair_sum(Red &red, const ItemOut &o);

__device__ __forceinline__ void finish_pair(Red &red, const ItemOut &o, const float (&acc0)[16],
                                            const float (&acc1)[16], const LaneRole &ln, int wave) {
    if (ln.useful) {
        float *dst0 = &red[0][wave][ln.gB][32 * ln.T + 16 * ln.h];
        float *dst1 = &red[1][wave][ln.gB][32 * ln.T + 16 * ln.h];
#pragma unroll
        for (int n = 0; n < 16; ++n) {
            dst0[n] = acc0[n];
            dst1[n] = acc1[n];
        }
    }
    finish_pair_sum<kStepGroups>(red, o);
}

template <int G>
__device__ __forceinline__ void finish_pair_sum(Red &red, const ItemOut &o) {
    __syncthreads();
    if (threadIdx.x < 2 * kBlockRows) {
        const uint32_t rb = threadIdx.x / kBlockRows, r = threadIdx.x % kBlockRows;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
#pragma unroll
            for (int g = 0; g < G; ++g) v += red[rb][w][g][r];
        const uint32_t row = o.block * 2 * kBlockRows + threadIdx.x;
        if (row < o.rows) {
            if (o.add != nullptr) v += ((gptr_cf32)o.add)[row];
            __builtin_nontemporal_store(v, (gptr_f32)o.y + row);
        }
    }
}

// VALU formulation: each lane's sums over its groups, reduced over the
// lanes sharing lane & 7 (lane l then holds row 4 (l & 7) + (l >> 4) of row
// tile T), published as red[s][wave][0][32 T + row].
__device__ __forceinline__ void publish_valu(float (&dst)[kWaves][kStepGroups][kBlockRows], const float (&acc)[2][4],
                                             int wave, int lane) {
#pragma unroll
    for (int T = 0; T < 2; ++T) {
        const float tot = add_over_a4(acc[T]);
        if ((lane & 8) == 0) dst[wave][0][32 * T + 4 * (lane & 7) + (lane >> 4)] = tot;
    }
}

// Registers of one full wave step at group g (t0 / t1 = group g of the
// block's two row tiles): the eight tiles' code bytes as restage() takes
// them, the lane's scales, digits and factor.
__device__ __forceinline__ void load_step_regs(WaveRegs &r, const uint8_t *t0, const uint8_t *t1, const uint8_t *prep,
                                               uint32_t g, const LaneRole &ln, int lane) {
#pragma unroll
    for (int c = 0; c < 8; ++c)
        r.code[c] = __builtin_nontemporal_load((gptr_i32x4)(((c & 1) ? t1 : t0) + (c >> 1) * kTileBytes + 64 + 16 * lane));
    const uint8_t *own = (ln.T ? t1 : t0) + ln.gB * kTileBytes + 32 * ln.h;
    r.sc[0] = __builtin_nontemporal_load((gptr_i32x4)own);
    r.sc[1] = __builtin_nontemporal_load((gptr_i32x4)(own + 16));
    r.a = *(gptr_i32x4)(prep + static_cast<size_t>(g + ln.gB) * kPrepBytes + ln.a_offset);
    r.f = *(gptr_cf32)(prep + static_cast<size_t>(g + ln.kslot) * kPrepBytes + 256);
}

// The wave's steps of one item: rt0 / rt1 = the block's two row tiles.
// Full step t reads groups g_begin + 16t + 4*wave .. +3; the rest up to
// g_end (fewer than 16 groups) is a short tail.  Each step's loads are
// issued after the previous step's arithmetic, so a wave has one step in
// flight: with two workgroups per CU that keeps about 12 MB in flight
// across the chip, and measured faster than two steps in flight (more
// outstanding loads only queue in the memory system once HBM is near its
// rate).
__device__ __forceinline__ void item_steps(const uint8_t *rt0, const uint8_t *rt1, const uint8_t *prep,
                                           uint32_t g_begin, uint32_t g_end, int wave, int lane, const LaneRole &ln,
                                           uint8_t *stage, float (&acc)[16], WaveRegs &pre, bool have_pre) {
    const uint32_t steps = (g_end - g_begin) / kWgStepGroups;
    uint32_t t = 0;
    if (have_pre) {
        // Step 0 was loaded into registers across the previous item's end.
        restage(pre, stage, ln, lane);
        compute_wave<false>(pre, acc, true);
        wait_lds_all();
        t = 1;
    }
    for (; t < steps; ++t) {
        const uint32_t g = g_begin + kWgStepGroups * t + kStepGroups * wave;
        const uint8_t *t0 = rt0 + static_cast<size_t>(g) * kTileBytes;
        const uint8_t *t1 = rt1 + static_cast<size_t>(g) * kTileBytes;
        // The eight tiles go straight to the wave's stage, where restage()
        // would have put them; scales and digits go to registers.
#pragma unroll
        for (int c = 0; c < 8; ++c) code_to_lds(((c & 1) ? t1 : t0) + (c >> 1) * kTileBytes, stage + kStageStride * c, lane);
        WaveRegs r;
        const uint8_t *own = (ln.T ? t1 : t0) + ln.gB * kTileBytes + 32 * ln.h;
        r.sc[0] = __builtin_nontemporal_load((gptr_i32x4)own);
        r.sc[1] = __builtin_nontemporal_load((gptr_i32x4)(own + 16));
        r.a = *(gptr_i32x4)(prep + static_cast<size_t>(g + ln.gB) * kPrepBytes + ln.a_offset);
        r.f = *(gptr_cf32)(prep + static_cast<size_t>(g + ln.kslot) * kPrepBytes + 256);
        wait_vm_all();
#pragma unroll
        for (int c = 0; c < 8; ++c) r.code[c] = *reinterpret_cast<const i32x4 *>(stage + ln.lds_read + 128 * c);
        compute_wave<false>(r, acc, true);
        wait_lds_all();  // every read of the stage is done before the next step's loads into it
    }
    // The short tail: the step's four groups are clamped to the chunk for
    // the loads, and those past its end are masked out.
    for (uint32_t g = g_begin + steps * kWgStepGroups + kStepGroups * wave; g < g_end; g += kWgStepGroups) {
        const uint32_t gb = min(g + ln.gB, g_end - 1);
        const uint32_t gf = g + ln.kslot;
        WaveRegs rr;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint32_t gc = min(g + (c >> 1), g_end - 1);
            const uint8_t *tile = ((c & 1) ? rt1 : rt0) + static_cast<size_t>(gc) * kTileBytes;
            rr.code[c] = __builtin_nontemporal_load((gptr_i32x4)(tile + 64 + 16 * lane));
        }
        const uint8_t *own = (ln.T ? rt1 : rt0) + static_cast<size_t>(gb) * kTileBytes + 32 * ln.h;
        rr.sc[0] = __builtin_nontemporal_load((gptr_i32x4)own);
        rr.sc[1] = __builtin_nontemporal_load((gptr_i32x4)(own + 16));
        rr.a = *(gptr_i32x4)(prep + static_cast<size_t>(gb) * kPrepBytes + ln.a_offset);
        rr.f = *(gptr_cf32)(prep + static_cast<size_t>(min(gf, g_end - 1)) * kPrepBytes + 256);
        restage(rr, stage, ln, lane);
        compute_wave<true>(rr, acc, gf < g_end);
    }
}

// Item `local` of GEMV d, decoded.  A SwiGLU GEMV whose rows fit one chunk
// (d.per == 1, two streams) streams W and then the gate over the same block
// in one item and applies the epilogue itself; a pair item streams its two
// 64-row blocks one after the other; otherwise an item is one stream's
// chunk and a block's items meet in the arrival chain.  rt[0..1] are the
// row tiles of the first pass, rt[2..3] those of the second (pair and
// both-streams items).  BOTH: the plan has both-streams GEMVs (the sweep
// without them is built without that path).
enum : uint32_t { kOnePass = 0, kPairPass = 1, kBothPass = 2 };
struct ItemCtx {
    const uint8_t *rt[4];
    const uint8_t *prep;
    uint32_t g_begin, g_end, kind;
    ItemOut o;
};

template <bool BOTH>
__device__ __forceinline__ ItemCtx decode_item(const PlanDesc &d, uint32_t local) {
    ItemCtx c;
    const uint32_t groups = d.cols / kGroup;
    const uint32_t tiles = d.rows / kTileRows;
    const size_t row_tile_bytes = static_cast<size_t>(groups) * kTileBytes;
    c.prep = d.prep;
    if (d.pair) {
        // Row tiles 4*local .. +3 (those past the last re-read the last;
        // their rows are never written), one K chunk.
#pragma unroll
        for (int i = 0; i < 4; ++i) c.rt[i] = d.w + static_cast<size_t>(min(4 * local + i, tiles - 1)) * row_tile_bytes;
        c.g_begin = 0;
        c.g_end = groups;
        c.kind = kPairPass;
        c.o = ItemOut{d.add, d.y, nullptr, nullptr, d.rows, local, 0, 1, 1, 1};
        return c;
    }
    const uint32_t per = d.per;  // items of one 64-row block
    const uint32_t block = local / per, part = local - block * per;
    const bool both = BOTH && d.streams > 1 && per == 1;
    const uint32_t stream = both ? 0 : part / d.chunks, chunk = both ? 0 : part - stream * d.chunks;
    c.g_begin = chunk * kChunkGroups;
    c.g_end = min(groups, c.g_begin + kChunkGroups);
    // The second row tile of a block past the last one re-reads the last
    // (its rows are never written).
    const size_t block_offset = static_cast<size_t>(2 * block) * row_tile_bytes;
    const size_t second = 2 * block + 1 < tiles ? row_tile_bytes : 0;
    c.rt[0] = (stream != 0 ? d.gate : d.w) + block_offset;
    c.rt[1] = c.rt[0] + second;
    c.rt[2] = both ? d.gate + block_offset : c.rt[0];
    c.rt[3] = c.rt[2] + second;
    c.kind = both ? kBothPass : kOnePass;
    c.o = ItemOut{d.add, d.y, d.partial, d.counters, d.rows, block, part, per, d.chunks, d.streams};
    return c;
}

#if defined(Q4RDNA_SWEEP_CLOCKS)
__device__ uint64_t g_sweep_clocks[2 * kMaxSweepClocks];
#endif

// Persistent grid: workgroup b runs the items the plan dealt it, entries
// [deal[b], deal[b + 1]) of the (descriptor, item within it) pairs that
// follow the gridDim.x + 1 offsets (padded to an even count), longest GEMVs
// first, as the plan orders them.  A fixed deal measured faster than an atomic item queue: while the
// sweep is bandwidth-bound, workgroups that finish early leave the others
// more of the bandwidth, and the queue's claim costs every item.
// Across an item's end (the barrier, the reduction and the stores) each
// wave already has the next item's first step in flight, in registers: the
// end would otherwise leave the workgroup with no loads outstanding.
template <bool BOTH>
__global__ __launch_bounds__(256) void plan_kernel(const PlanDesc *__restrict__ descs,
                                                   const uint32_t *__restrict__ deal) {
    __shared__ Shared sh;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#if defined(Q4RDNA_SWEEP_CLOCKS)
    const uint64_t clock_start = __builtin_amdgcn_s_memrealtime();
#endif
    const LaneRole ln = lane_role(lane);
    const uint2 *entry = reinterpret_cast<const uint2 *>(deal + ((gridDim.x + 2) & ~1u));
    const uint32_t end = deal[blockIdx.x + 1];
    uint32_t k = deal[blockIdx.x];
    if (k >= end) return;
    auto locate = [&](uint2 e) { return decode_item<BOTH>(descs[e.x], e.y); };
    ItemCtx cur = locate(entry[k]);
    WaveRegs pre;
    bool have_pre = false;
    uint32_t parity = 0;
    for (;;) {
        // The next entry is read now, so that only its descriptor's loads
        // stand between this item's last step and the next item's loads.
        const uint2 next_entry = k + 1 < end ? entry[k + 1] : make_uint2(0, 0);
        float acc[16], acc1[16];
#pragma unroll
        for (int n = 0; n < 16; ++n) acc[n] = acc1[n] = 0.0f;
        item_steps(cur.rt[0], cur.rt[1], cur.prep, cur.g_begin, cur.g_end, wave, lane, ln, sh.stage[wave], acc, pre,
                   have_pre);
        if (cur.kind != kOnePass)
            item_steps(cur.rt[2], cur.rt[3], cur.prep, cur.g_begin, cur.g_end, wave, lane, ln, sh.stage[wave], acc1,
                       pre, false);
        ++k;
        ItemCtx next;
        have_pre = false;
        if (k < end) {
            next = locate(next_entry);
            if (next.g_end - next.g_begin >= kWgStepGroups) {
                const uint32_t g = next.g_begin + kStepGroups * wave;
                load_step_regs(pre, next.rt[0] + static_cast<size_t>(g) * kTileBytes,
                               next.rt[1] + static_cast<size_t>(g) * kTileBytes, next.prep, g, ln, lane);
                have_pre = true;
            }
        }
        Red &red = sh.red[parity];
        parity ^= 1;
        if (cur.kind == kPairPass)
            finish_pair(red, cur.o, acc, acc1, ln, wave);
        else if (BOTH && cur.kind == kBothPass)
            finish_item<true>(red, sh.last, cur.o, acc, acc1, ln, wave);
        else
            finish_item<false>(red, sh.last, cur.o, acc, acc1, ln, wave);
        if (k >= end) break;
        cur = next;
    }
#if defined(Q4RDNA_SWEEP_CLOCKS)
    // After the last item's stores have left: this workgroup's end.
    __syncthreads();
    if (threadIdx.x == 0 && blockIdx.x < kMaxSweepClocks) {
        const uint64_t clock_end = __builtin_amdgcn_s_memrealtime();
        g_sweep_clocks[2 * blockIdx.x] = clock_start;
        g_sweep_clocks[2 * blockIdx.x + 1] = clock_end;
    }
#endif
}

// ---- the sweep in the VALU formulation (kSweepValu) -------------------------
//
// plan_kernel's items, deal, loads and finish with compute_valu's arithmetic:
// each step's eight tiles go straight to the wave's LDS stage as in the
// MFMA sweep, scales and prepared x to registers; one step in flight; the
// next item's first step loaded across an item's end.

__device__ __forceinline__ void stage_codes(const i32x4 (&code)[8], uint8_t *stage, int lane) {
#pragma unroll
    for (int c = 0; c < 8; ++c) *reinterpret_cast<i32x4 *>(stage + kStageStride * c + 16 * lane) = code[c];
    __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ void load_step_valu(ValuRegs &r, const uint8_t *rt0, const uint8_t *rt1, const uint8_t *prep,
                                               uint32_t g, uint32_t g_last, int lane) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const uint32_t gc = min(g + (c >> 1), g_last);
        r.code[c] = __builtin_nontemporal_load(
            (gptr_i32x4)(((c & 1) ? rt1 : rt0) + static_cast<size_t>(gc) * kTileBytes + 64 + 16 * lane));
    }
    load_valu_aux(r.aux, rt0, rt1, prep, g, g_last, lane & 7, lane >> 3);
}

__device__ __forceinline__ void item_steps_valu(const uint8_t *rt0, const uint8_t *rt1, const uint8_t *prep,
                                                uint32_t g_begin, uint32_t g_end, int wave, int lane, uint8_t *stage,
                                                float (&acc)[2][4], ValuRegs &pre, bool have_pre) {
    const int q = lane & 7, a = lane >> 3;
    const uint32_t steps = (g_end - g_begin) / kWgStepGroups;
    uint32_t t = 0;
    if (have_pre) {
        stage_codes(pre.code, stage, lane);
        compute_valu<false>(stage, pre.aux, acc, q, a, kStepGroups);
        wait_lds_all();
        t = 1;
    }
    for (; t < steps; ++t) {
        const uint32_t g = g_begin + kWgStepGroups * t + kStepGroups * wave;
#pragma unroll
        for (int c = 0; c < 8; ++c)
            code_to_lds(((c & 1) ? rt1 : rt0) + static_cast<size_t>(g + (c >> 1)) * kTileBytes, stage + kStageStride * c,
                        lane);
        ValuAux r;
        load_valu_aux(r, rt0, rt1, prep, g, g_end - 1, q, a);
        wait_vm_all();
        compute_valu<false>(stage, r, acc, q, a, kStepGroups);
        wait_lds_all();  // every read of the stage is done before the next step's loads into it
    }
    for (uint32_t g = g_begin + steps * kWgStepGroups + kStepGroups * wave; g < g_end; g += kWgStepGroups) {
        ValuRegs rr;
        load_step_valu(rr, rt0, rt1, prep, g, g_end - 1, lane);
        stage_codes(rr.code, stage, lane);
        compute_valu<true>(stage, rr.aux, acc, q, a, g_end - g);
        wait_lds_all();
    }
}

template <bool BOTH>
__global__ __launch_bounds__(256) void plan_valu_kernel(const PlanDesc *__restrict__ descs,
                                                        const uint32_t *__restrict__ deal) {
    __shared__ Shared sh;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint2 *entry = reinterpret_cast<const uint2 *>(deal + ((gridDim.x + 2) & ~1u));
    const uint32_t end = deal[blockIdx.x + 1];
    uint32_t k = deal[blockIdx.x];
    if (k >= end) return;
    auto locate = [&](uint2 e) { return decode_item<BOTH>(descs[e.x], e.y); };
    ItemCtx cur = locate(entry[k]);
    ValuRegs pre;
    bool have_pre = false;
    uint32_t parity = 0;
    for (;;) {
        const uint2 next_entry = k + 1 < end ? entry[k + 1] : make_uint2(0, 0);
        float acc[2][4] = {}, acc1[2][4] = {};
        item_steps_valu(cur.rt[0], cur.rt[1], cur.prep, cur.g_begin, cur.g_end, wave, lane, sh.stage[wave], acc, pre,
                        have_pre);
        if (cur.kind != kOnePass)
            item_steps_valu(cur.rt[2], cur.rt[3], cur.prep, cur.g_begin, cur.g_end, wave, lane, sh.stage[wave], acc1,
                            pre, false);
        ++k;
        ItemCtx next;
        have_pre = false;
        if (k < end) {
            next = locate(next_entry);
            if (next.g_end - next.g_begin >= kWgStepGroups) {
                load_step_valu(pre, next.rt[0], next.rt[1], next.prep, next.g_begin + kStepGroups * wave,
                               next.g_end - 1, lane);
                have_pre = true;
            }
        }
        Red &red = sh.red[parity];
        parity ^= 1;
        publish_valu(red[0], acc, wave, lane);
        if (cur.kind != kOnePass) publish_valu(red[1], acc1, wave, lane);
        if (cur.kind == kPairPass)
            finish_pair_sum<1>(red, cur.o);
        else if (BOTH && cur.kind == kBothPass)
            finish_item_sum<true, 1>(red, sh.last, cur.o);
        else
            finish_item_sum<false, 1>(red, sh.last, cur.o);
        if (k >= end) break;
        cur = next;
    }
}

// ---- batched sweep (N = 2..8 activation vectors) ---------------------------
//
// With several activation vectors the A operand's rows carry the vectors
// instead of groups: one MFMA multiplies 16 row sets of ONE group by the
// three digits of up to four vectors (rows 4n + d of A, d = 3 unused), so
// every lane of D is useful for N = 4 and a second vector quad costs one more
// MFMA per operand, not more loads or transposes.
//  * Item: (256-row block = 8 row tiles, stream, K chunk of up to
//    kBatchChunkGroups = 192 groups); wave w takes groups
//    chunk start + w + 4s, one per step.  A SwiGLU GEMV whose rows fit one
//    chunk has one item per block that streams up and then gate.
//  * Loads per step: load instruction c reads the whole code area of row
//    tile c at the step's group (1 KB contiguous), restaged through LDS as in
//    the single-vector sweep; lane (kslot, j) then reads rows 16h..16h+15 of
//    row tile T = j/2, h = j%2, at k-pairs kslot + 4c.
//  * D: lane l holds D rows 4*(l/16)..+3 of column j = l%16, i.e. vector
//    l/16 of the quad, digits 0..2, for the 16 rows of column j; it loads
//    those rows' scales and the vector's group factor itself.
// Prep layout per (group, vector quad), kBatchQuadBytes = 1040: digit d of
// vector n at byte kslot*256 + (4n + d)*16 + e (the operand order above),
// then the four vectors' group factors at 1024.
constexpr int kBatchRows = 256;
constexpr uint32_t kBatchQuadBytes = 1040;

// Lane 4p + kslot of a wave converts k-slot kslot of the wave's (group,
// vector) pair p (16 pairs per wave, pair = g * n + vector).  Slots past n in
// the last quad are never written and stay zero from the plan's creation.
// PAD: whole records (n > 2).  Whole records measured faster at n = 4 and 8
// (prepare 15 / 25 against 17 / 31 us) and slower at n = 2 (12.5 against
// 10.4 us), where half of each quad's slots stay unwritten anyway.  As a
// run-time flag the same choice measured slower at n = 4 and 8 (21 / 38 us).
template <bool PAD>
__global__ __launch_bounds__(256) void prep_batch_kernel(const PlanDesc *__restrict__ descs,
                                                         const uint32_t *__restrict__ owner, uint32_t total_groups,
                                                         uint32_t n) {
    const int lane = threadIdx.x & 63, kslot = lane & 3;
    const uint32_t pair = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 16 + (lane >> 2);
    const bool valid = pair < total_groups * n;
    const uint32_t pq = valid ? pair : 0;
    const uint32_t gid = pq / n, vec = pq - gid * n;
    const PlanDesc &d = descs[owner[gid]];
    const uint32_t g = gid - d.group_begin;
    const uint32_t quads = (n + 3) / 4, slot = vec & 3;
    const float *x = d.x + static_cast<size_t>(vec) * d.cols + static_cast<size_t>(g) * kGroup;
    gptr_u8 quad = (gptr_u8)(d.prep + (static_cast<size_t>(g) * quads + vec / 4) * kBatchQuadBytes);
    bool bad;
    int e;
    prep_kslot(x, kslot, valid, PAD, quad + 256 * kslot + 64 * slot, bad, e);
    if (valid && kslot == 0) __builtin_nontemporal_store(digit_factor(bad, e), (gptr_f32)(quad + 1024 + 4 * slot));
}

constexpr int kBatchWaves = 4;  // eight waves per workgroup measured slower

// A wave's stage also receives its partial sums at the item's end (after
// its last step, so the two uses never overlap): 4*NQ x 256 floats <= 8 KB.
template <int NQ>
struct BatchShared {
    uint8_t stage[kBatchWaves][kStageBytes];
    uint32_t next_item[2];
    uint32_t last;
};
static_assert(8 * kBatchRows * sizeof(float) <= kStageBytes, "partials must fit a wave's stage");

struct BatchRegs {
    i32x4 code[8];
    i32x4 sc[2];
};

template <int NQ>
__device__ __forceinline__ void compute_batch(const BatchRegs &r, const i32x4 (&a)[NQ], const float (&f)[NQ],
                                              float (&acc)[NQ][16]) {
    const i32x4 zero = {0, 0, 0, 0};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        uint32_t t[8];
        transpose4(r.code[0][m], r.code[1][m], r.code[2][m], r.code[3][m], t[0], t[1], t[2], t[3]);
        transpose4(r.code[4][m], r.code[5][m], r.code[6][m], r.code[7][m], t[4], t[5], t[6], t[7]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int n = 4 * m + q;
            i32x4 b;
            b[0] = static_cast<int>(low_nibbles_x16(t[q]));
            b[1] = static_cast<int>(high_nibbles_x16(t[q]));
            b[2] = static_cast<int>(low_nibbles_x16(t[4 + q]));
            b[3] = static_cast<int>(high_nibbles_x16(t[4 + q]));
            const uint32_t word = static_cast<uint32_t>(r.sc[n >> 3][(n >> 1) & 3]);
            const float s = half_bits_to_float((n & 1) ? (word >> 16) : word);
#pragma unroll
            for (int vq = 0; vq < NQ; ++vq) {
                const i32x4 dm = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[vq], b, zero, 0, 0, 0);
                const int d01 = dm[0] + (dm[1] << 8);
                const float v = fmaf(static_cast<float>(dm[2]), 65536.0f, static_cast<float>(d01));
                acc[vq][n] = fmaf(s * f[vq], v, acc[vq][n]);
            }
        }
    }
}

template <int NQ>
__device__ __forceinline__ void run_batch_item(BatchShared<NQ> &sh, const PlanDesc &d, uint32_t local, uint32_t nvec,
                                               int lane, int wave) {
    const uint32_t groups = d.cols / kGroup;
    const uint32_t tiles = d.rows / kTileRows;
    const uint32_t per = d.per;
    // A SwiGLU GEMV whose rows fit one chunk has one item per block that
    // streams up, then gate, into two accumulator sets (no partials).
    const bool both = d.streams > 1 && per == 1;
    const uint32_t block = local / per, part = local - block * per;
    const uint32_t stream = part / d.chunks, chunk = part - stream * d.chunks;
    const uint32_t g_begin = chunk * kBatchChunkGroups;
    const uint32_t g_end = min(groups, g_begin + kBatchChunkGroups);
    const size_t row_tile_bytes = static_cast<size_t>(groups) * kTileBytes;
    const uint8_t *base = stream != 0 ? d.gate : d.w;
    const int kslot = lane >> 4, j = lane & 15, T = j >> 1, h = j & 1;
    const uint32_t lds_read = kStageStride * T + 32 * kslot + 16 * h;
    // The block's eight row tiles; those past the last re-read the last
    // (their rows are never written).
    const uint8_t *rt[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) rt[c] = base + static_cast<size_t>(min(8 * block + c, tiles - 1)) * row_tile_bytes;
    const size_t prep_stride = static_cast<size_t>(NQ) * kBatchQuadBytes;
    float acc[NQ][16];
#pragma unroll
    for (int vq = 0; vq < NQ; ++vq)
#pragma unroll
        for (int n = 0; n < 16; ++n) acc[vq][n] = 0.0f;

    auto load = [&](uint32_t g, BatchRegs &r) {
#pragma unroll
        for (int c = 0; c < 8; ++c)
            r.code[c] = __builtin_nontemporal_load((gptr_i32x4)(rt[c] + static_cast<size_t>(g) * kTileBytes + 64 + 16 * lane));
        const uint8_t *own = rt[T] + static_cast<size_t>(g) * kTileBytes + 32 * h;
        r.sc[0] = __builtin_nontemporal_load((gptr_i32x4)own);
        r.sc[1] = __builtin_nontemporal_load((gptr_i32x4)(own + 16));
        __builtin_amdgcn_sched_barrier(0);
    };
    auto step = [&](uint32_t g, BatchRegs &r) {
        i32x4 a[NQ];
        float f[NQ];
        const uint8_t *pg = d.prep + static_cast<size_t>(g) * prep_stride;
#pragma unroll
        for (int vq = 0; vq < NQ; ++vq) {
            a[vq] = *(gptr_i32x4)(pg + vq * kBatchQuadBytes + 256 * kslot + 16 * j);
            f[vq] = *(gptr_cf32)(pg + vq * kBatchQuadBytes + 1024 + 4 * kslot);
        }
        // Restaged through registers: loading straight into LDS, as the
        // single-vector sweep does, measured neutral to 0.6 % slower here.
#pragma unroll
        for (int c = 0; c < 8; ++c) *reinterpret_cast<i32x4 *>(sh.stage[wave] + kStageStride * c + 16 * lane) = r.code[c];
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int c = 0; c < 8; ++c) r.code[c] = *reinterpret_cast<const i32x4 *>(sh.stage[wave] + lds_read + 128 * c);
        compute_batch<NQ>(r, a, f, acc);
    };
    // One step in flight per wave: each step's loads follow the previous
    // step's arithmetic (two steps in flight measured slower, as in the
    // single-vector sweep).  Loading the next item's first step across this
    // item's end, after the barrier that follows the last step (the next
    // item is claimed one ahead), measured 0.6-1.3 % slower at N = 2, 4, 8.
    // Lane (kslot, j) holds vector 4*vq + kslot, rows 32T + 16h + n; the
    // wave's partials go to red[vector][row] in its own stage.
    float *red = reinterpret_cast<float *>(sh.stage[wave]);
    auto publish = [&]() {
#pragma unroll
        for (int vq = 0; vq < NQ; ++vq) {
            const uint32_t vec = 4 * vq + kslot;
            if (vec < nvec) {
                float *dst = red + (4 * vq + kslot) * kBatchRows + 32 * T + 16 * h;
#pragma unroll
                for (int n = 0; n < 16; ++n) dst[n] = acc[vq][n];
            }
        }
    };
    // Threads split the block's rows; each sums its rows' partials over the
    // waves in wave order.
    auto total = [&](uint32_t vec, uint32_t r) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kBatchWaves; ++w) v += reinterpret_cast<const float *>(sh.stage[w])[vec * kBatchRows + r];
        return v;
    };

    for (uint32_t g = g_begin + wave; g < g_end; g += kBatchWaves) {
        BatchRegs r;
        load(g, r);
        step(g, r);
    }
    // Both streams: the up sums go to registers, one row per thread
    // (blockDim.x == kBatchRows), and the accumulators start over on the gate.
    constexpr int V = 4 * NQ;
    float u[V];
    if (both) {
        publish();
        __syncthreads();
#pragma unroll
        for (int vec = 0; vec < V; ++vec) u[vec] = static_cast<uint32_t>(vec) < nvec ? total(vec, threadIdx.x) : 0.0f;
        __syncthreads();
#pragma unroll
        for (int vq = 0; vq < NQ; ++vq)
#pragma unroll
            for (int n = 0; n < 16; ++n) acc[vq][n] = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; ++c)
            rt[c] = d.gate + static_cast<size_t>(min(8 * block + c, tiles - 1)) * row_tile_bytes;
        for (uint32_t g = g_begin + wave; g < g_end; g += kBatchWaves) {
            BatchRegs r;
            load(g, r);
            step(g, r);
        }
    }
    publish();
    __syncthreads();
    const size_t M = d.rows;
    if (both) {
        // y = (up + add) * silu(gate), the up sums from registers.
        const uint32_t r = threadIdx.x, row = block * kBatchRows + r;
        if (row < d.rows) {
#pragma unroll
            for (int vec = 0; vec < V; ++vec) {
                if (static_cast<uint32_t>(vec) >= nvec) break;
                float v = u[vec];
                if (d.add != nullptr) v += ((gptr_cf32)d.add)[vec * M + row];
                __builtin_nontemporal_store(v * silu(total(vec, r)), (gptr_f32)d.y + vec * M + row);
            }
        }
        return;
    }
    if (per == 1) {
        for (uint32_t r = threadIdx.x; r < kBatchRows; r += blockDim.x) {
            const uint32_t row = block * kBatchRows + r;
            if (row >= d.rows) break;
            for (uint32_t vec = 0; vec < nvec; ++vec) {
                float v = total(vec, r);
                if (d.add != nullptr) v += ((gptr_cf32)d.add)[vec * M + row];
                __builtin_nontemporal_store(v, (gptr_f32)d.y + vec * M + row);
            }
        }
        return;
    }
    for (uint32_t r = threadIdx.x; r < kBatchRows; r += blockDim.x) {
        const uint32_t row = block * kBatchRows + r;
        if (row >= d.rows) break;
        for (uint32_t vec = 0; vec < nvec; ++vec)
            store_agent(&d.partial[(static_cast<size_t>(part) * nvec + vec) * M + row], total(vec, r));
    }
    wait_stores();
    __syncthreads();
    if (threadIdx.x == 0) sh.last = (add_agent(&d.counters[block], 1u) == per - 1) ? 1u : 0u;
    __syncthreads();
    if (sh.last == 0u) return;
    for (uint32_t r = threadIdx.x; r < kBatchRows; r += blockDim.x) {
        const uint32_t row = block * kBatchRows + r;
        if (row >= d.rows) break;
        for (uint32_t vec = 0; vec < nvec; ++vec) {
            float u = load_agent(&d.partial[static_cast<size_t>(vec) * M + row]);
            for (uint32_t k = 1; k < d.chunks; ++k) u += load_agent(&d.partial[(static_cast<size_t>(k) * nvec + vec) * M + row]);
            if (d.add != nullptr) u += ((gptr_cf32)d.add)[vec * M + row];
            if (d.streams > 1) {
                float g = load_agent(&d.partial[(static_cast<size_t>(d.chunks) * nvec + vec) * M + row]);
                for (uint32_t k = 1; k < d.chunks; ++k)
                    g += load_agent(&d.partial[(static_cast<size_t>(d.chunks + k) * nvec + vec) * M + row]);
                u *= silu(g);
            }
            __builtin_nontemporal_store(u, (gptr_f32)d.y + vec * M + row);
        }
    }
    if (threadIdx.x == 0) store_agent(&d.counters[block], 0u);
}

template <int NQ>
__global__ __launch_bounds__(64 * kBatchWaves) void plan_batch_kernel(const PlanDesc *__restrict__ descs, uint32_t items,
                                                         uint32_t nvec, uint32_t *__restrict__ sched) {
    __shared__ BatchShared<NQ> sh;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#if defined(Q4RDNA_SWEEP_CLOCKS)
    const uint64_t clock_start = __builtin_amdgcn_s_memrealtime();
#endif
    if (threadIdx.x == 0) sh.next_item[0] = add_agent(&sched[0], 1u);
    __syncthreads();
    uint32_t item = sh.next_item[0];
    uint32_t d = 0;
    int slot = 0;
    while (item < items) {
        if (threadIdx.x == 0) sh.next_item[slot ^ 1] = add_agent(&sched[0], 1u);
        while (item >= descs[d + 1].item_begin) ++d;
        run_batch_item<NQ>(sh, descs[d], item - descs[d].item_begin, nvec, lane, wave);
        __syncthreads();
        slot ^= 1;
        item = sh.next_item[slot];
    }
#if defined(Q4RDNA_SWEEP_CLOCKS)
    // After the last item (the loop ends at a barrier that follows it).
    if (threadIdx.x == 0 && blockIdx.x < kMaxSweepClocks) {
        const uint64_t clock_end = __builtin_amdgcn_s_memrealtime();
        g_sweep_clocks[2 * blockIdx.x] = clock_start;
        g_sweep_clocks[2 * blockIdx.x + 1] = clock_end;
    }
#endif
    if (threadIdx.x == 0 && add_agent(&sched[1], 1u) == gridDim.x - 1) {
        store_agent(&sched[0], 0u);
        store_agent(&sched[1], 0u);
    }
}

}  // namespace

#if defined(Q4RDNA_SWEEP_CLOCKS)
}  // namespace q4rdna
// Clock build only: the latest sweep's per-workgroup (start, end) clocks,
// 2 * count values for workgroups 0..count-1 (count <= kMaxSweepClocks).
extern "C" int q4rdna_sweep_clocks(uint64_t *out, uint32_t count) {
    if (out == nullptr || count > q4rdna::kMaxSweepClocks) return -1;
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(q4rdna::g_sweep_clocks), 2 * sizeof(uint64_t) * count, 0,
                               hipMemcpyDeviceToHost) == hipSuccess ? 0 : -4;
}
namespace q4rdna {
#endif

hipError_t launch_prep(const float *const *group_x, uint8_t *prep, uint32_t groups, hipStream_t stream) {
    if (groups == 0) return hipSuccess;
    if constexpr (kSweepValu)
        hipLaunchKernelGGL(prep_valu_kernel, dim3((groups * 8 + 255) / 256), dim3(256), 0, stream, group_x, prep,
                           groups);
    else
        hipLaunchKernelGGL(prep_kernel, dim3((groups + 63) / 64), dim3(256), 0, stream, group_x, prep, groups);
    return hipGetLastError();
}

hipError_t launch_plan(const PlanDesc *descs, const uint32_t *deal, uint32_t workgroups, bool both_streams,
                       hipStream_t stream) {
    if constexpr (kSweepValu) {
        if (both_streams)
            hipLaunchKernelGGL(plan_valu_kernel<true>, dim3(workgroups), dim3(256), 0, stream, descs, deal);
        else
            hipLaunchKernelGGL(plan_valu_kernel<false>, dim3(workgroups), dim3(256), 0, stream, descs, deal);
    } else {
        if (both_streams)
            hipLaunchKernelGGL(plan_kernel<true>, dim3(workgroups), dim3(256), 0, stream, descs, deal);
        else
            hipLaunchKernelGGL(plan_kernel<false>, dim3(workgroups), dim3(256), 0, stream, descs, deal);
    }
    return hipGetLastError();
}

hipError_t launch_prep_batch(const PlanDesc *descs, const uint32_t *owner, uint32_t groups, uint32_t n,
                             hipStream_t stream) {
    if (groups == 0) return hipSuccess;
    if (n > 2)
        hipLaunchKernelGGL(prep_batch_kernel<true>, dim3((groups * n + 63) / 64), dim3(256), 0, stream, descs, owner,
                           groups, n);
    else
        hipLaunchKernelGGL(prep_batch_kernel<false>, dim3((groups * n + 63) / 64), dim3(256), 0, stream, descs, owner,
                           groups, n);
    return hipGetLastError();
}

hipError_t launch_plan_batch(const PlanDesc *descs, uint32_t items, uint32_t n, uint32_t workgroups, uint32_t *sched,
                             hipStream_t stream) {
    const dim3 block(64 * kBatchWaves);
    if (n <= 4)
        hipLaunchKernelGGL(plan_batch_kernel<1>, dim3(workgroups), block, 0, stream, descs, items, n, sched);
    else
        hipLaunchKernelGGL(plan_batch_kernel<2>, dim3(workgroups), block, 0, stream, descs, items, n, sched);
    return hipGetLastError();
}

}  // namespace q4rdna
