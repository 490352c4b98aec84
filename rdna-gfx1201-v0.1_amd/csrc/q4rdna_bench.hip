// Measurement kernels for bench.py (libq4rdna_bench_gfx950.so).  They are not
// part of the GEMV library or its C ABI: they give the figures the GEMV
// kernels are compared with (a plain read of the same bytes, an empty
// launch) and the RMS normalization the decoder-layer bench puts between
// layers.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "q4rdna_device.h"

namespace {

constexpr int kReadThreads = 512;
constexpr int kReadLoads = 16;  // dword loads per thread, all in flight: 32 KB per workgroup
constexpr uint64_t kReadChunk = static_cast<uint64_t>(kReadThreads) * kReadLoads * 4;

// Workgroup b (remapped so consecutive chunks share an XCD) reads bytes
// [b * 32 KB, (b + 1) * 32 KB) with nontemporal dword loads, each load of a
// wave one contiguous 256-byte run; past the end the index is clamped, so
// every load is issued unconditionally.  The XOR of the data is stored only
// when `flag` is set and it equals a constant the caller never passes, so
// the loads cannot be dropped and nothing is written.
__global__ __launch_bounds__(kReadThreads) void stream_read_kernel(const uint32_t *__restrict__ p, uint64_t words,
                                                                   uint32_t *sink, uint32_t flag) {
    const uint64_t b = q4rdna::xcd_remap(blockIdx.x, gridDim.x);
    const uint64_t base = b * (kReadChunk / 4) + threadIdx.x;
    uint32_t v[kReadLoads];
#pragma unroll
    for (int i = 0; i < kReadLoads; ++i) {
        const uint64_t w = base + static_cast<uint64_t>(i) * kReadThreads;
        v[i] = __builtin_nontemporal_load((q4rdna::gptr_u32)(p + (w < words ? w : words - 1)));
    }
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < kReadLoads; ++i) acc ^= v[i];
    if (flag != 0 && acc == flag) sink[threadIdx.x] = acc;
}

// stream_read_kernel's read of `words` words at p by workgroups
// 0..own_blocks-1, plus a cache-allocating read of `twords` words at t (the
// bytes the next launch reads), which leaves them in the Infinity Cache:
//   * tloads > 0: each reading workgroup, after its own loads, reads its
//     tloads * 512-word slice of t (slice b of workgroup b);
//   * tloads == 0: workgroups own_blocks.. (dispatched after every reading
//     workgroup) read t in 32 KB chunks, 16 loads per thread.
// Indexes past either end are clamped, so every load is issued; the XOR of
// the data reaches `sink` only when it equals `flag`, which the caller never
// passes nonzero.
__global__ __launch_bounds__(kReadThreads) void stream_read_touch_kernel(const uint32_t *__restrict__ p,
                                                                         uint64_t words, uint32_t own_blocks,
                                                                         const uint32_t *__restrict__ t,
                                                                         uint64_t twords, uint32_t tloads,
                                                                         uint32_t *sink, uint32_t flag) {
    uint32_t acc = 0;
    if (blockIdx.x < own_blocks) {
        const uint64_t b = q4rdna::xcd_remap(blockIdx.x, own_blocks);
        const uint64_t base = b * (kReadChunk / 4) + threadIdx.x;
        uint32_t v[kReadLoads];
#pragma unroll
        for (int i = 0; i < kReadLoads; ++i) {
            const uint64_t w = base + static_cast<uint64_t>(i) * kReadThreads;
            v[i] = __builtin_nontemporal_load((q4rdna::gptr_u32)(p + (w < words ? w : words - 1)));
        }
        const uint64_t tbase = b * tloads * kReadThreads + threadIdx.x;
#pragma unroll 4
        for (uint32_t i = 0; i < tloads; ++i) {
            const uint64_t w = tbase + static_cast<uint64_t>(i) * kReadThreads;
            acc ^= t[w < twords ? w : twords - 1];
        }
#pragma unroll
        for (int i = 0; i < kReadLoads; ++i) acc ^= v[i];
    } else {
        const uint64_t base = static_cast<uint64_t>(blockIdx.x - own_blocks) * (kReadChunk / 4) + threadIdx.x;
        uint32_t v[kReadLoads];
#pragma unroll
        for (int i = 0; i < kReadLoads; ++i) {
            const uint64_t w = base + static_cast<uint64_t>(i) * kReadThreads;
            v[i] = t[w < twords ? w : twords - 1];
        }
#pragma unroll
        for (int i = 0; i < kReadLoads; ++i) acc ^= v[i];
    }
    if (flag != 0 && acc == flag) sink[threadIdx.x] = acc;
}

// The sweeps' access pattern, as a plain read: `gridDim.x` persistent
// workgroups of four waves, each wave with one step of eight 1 KB loads
// (64 lanes x 16 bytes, nontemporal) in flight at a time.  Workgroup b reads
// `lines` 1 KB lines from b * lines on as `runs` contiguous runs of
// lines / runs; load c of wave w in workgroup step s reads run
// (8w + c) % runs at line s * (32 / runs) + (8w + c) / runs.  runs = 2 is
// the single-vector sweep's pattern (two row tiles per workgroup, four
// consecutive groups per wave step), runs = 8 the batched sweep's (eight row
// tiles, one group per wave step).  lines is a multiple of 32 and runs
// divides 32; the XOR goes to `sink` only when it equals `flag`, which the
// caller never passes nonzero.
__global__ __launch_bounds__(256) void stream_runs_kernel(const uint8_t *__restrict__ p, uint32_t lines,
                                                          uint32_t runs, uint32_t *sink, uint32_t flag) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint8_t *base = p + static_cast<uint64_t>(blockIdx.x) * lines * 1024 + 16 * lane;
    const uint32_t run_lines = lines / runs, per_step = 32 / runs;
    uint32_t run_off[8], pos_off[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const uint32_t i = 8 * wave + c;
        run_off[c] = (i % runs) * run_lines;
        pos_off[c] = i / runs;
    }
    uint32_t acc = 0;
#pragma unroll 1
    for (uint32_t s = 0; s < lines / 32; ++s) {
        q4rdna::i32x4 v[8];
#pragma unroll
        for (int c = 0; c < 8; ++c)
            v[c] = __builtin_nontemporal_load(
                (q4rdna::gptr_i32x4)(base + static_cast<uint64_t>(run_off[c] + s * per_step + pos_off[c]) * 1024));
#pragma unroll
        for (int c = 0; c < 8; ++c) acc ^= static_cast<uint32_t>(v[c][0] ^ v[c][1] ^ v[c][2] ^ v[c][3]);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (flag != 0 && acc == flag) sink[threadIdx.x] = acc;
}

__global__ void empty_kernel() {}

// y = x * rsqrt(mean(x^2) + eps) by one workgroup of 1024 threads.
constexpr int kNormThreads = 1024;
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(const float *__restrict__ x, float *__restrict__ y,
                                                                uint32_t n, float eps) {
    __shared__ float part[kNormThreads / 64];
    float s = 0.f;
    for (uint32_t i = threadIdx.x; i < n; i += kNormThreads) s = fmaf(x[i], x[i], s);
    s = q4rdna::add_over_a(s);  // lanes sharing lane & 7
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < kNormThreads / 64; ++w) t += part[w];
    const float r = rsqrtf(t / static_cast<float>(n) + eps);
    for (uint32_t i = threadIdx.x; i < n; i += kNormThreads) y[i] = x[i] * r;
}

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 4, at least 4) at p once; sink is 512 words
// that are never written in practice.
int q4bench_stream_read(const void *p, uint64_t bytes, uint32_t *sink, hipStream_t stream) {
    if (p == nullptr || sink == nullptr || bytes < 4 || bytes % 4 != 0) return static_cast<int>(hipErrorInvalidValue);
    const uint64_t blocks = (bytes + kReadChunk - 1) / kReadChunk;
    if (blocks > 0x7fffffffull) return static_cast<int>(hipErrorInvalidValue);
    hipLaunchKernelGGL(stream_read_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kReadThreads), 0, stream,
                       static_cast<const uint32_t *>(p), bytes / 4, sink, 0u);
    return static_cast<int>(hipGetLastError());
}

// Reads `bytes` at p like q4bench_stream_read and `touch_bytes` at t with
// cache-allocating loads (both multiples of 4, at least 4): by the reading
// workgroups after their own loads when `inline_touch` is nonzero, else by
// workgroups appended to the launch.
int q4bench_stream_read_touch(const void *p, uint64_t bytes, const void *t, uint64_t touch_bytes, int inline_touch,
                              uint32_t *sink, hipStream_t stream) {
    if (p == nullptr || t == nullptr || sink == nullptr || bytes < 4 || bytes % 4 != 0 || touch_bytes < 4 ||
        touch_bytes % 4 != 0)
        return static_cast<int>(hipErrorInvalidValue);
    const uint64_t blocks = (bytes + kReadChunk - 1) / kReadChunk;
    const uint64_t touch_blocks = (touch_bytes + kReadChunk - 1) / kReadChunk;
    uint64_t tloads = 0, grid = blocks + touch_blocks;
    if (inline_touch != 0) {
        tloads = (touch_bytes / 4 + blocks * kReadThreads - 1) / (blocks * kReadThreads);
        grid = blocks;
    }
    if (grid > 0x7fffffffull || tloads > 4096) return static_cast<int>(hipErrorInvalidValue);
    hipLaunchKernelGGL(stream_read_touch_kernel, dim3(static_cast<uint32_t>(grid)), dim3(kReadThreads), 0, stream,
                       static_cast<const uint32_t *>(p), bytes / 4, static_cast<uint32_t>(blocks),
                       static_cast<const uint32_t *>(t), touch_bytes / 4, static_cast<uint32_t>(tloads), sink, 0u);
    return static_cast<int>(hipGetLastError());
}

// One launch of stream_runs_kernel: `workgroups` x 256 threads, each
// workgroup reading `lines` 1 KB lines as `runs` runs; the buffer at p must
// hold workgroups * lines KB.
int q4bench_stream_runs(const void *p, uint32_t workgroups, uint32_t lines, uint32_t runs, uint32_t *sink,
                        hipStream_t stream) {
    if (p == nullptr || sink == nullptr || workgroups == 0 || lines == 0 || lines % 32 != 0 || runs == 0 ||
        32 % runs != 0)
        return static_cast<int>(hipErrorInvalidValue);
    hipLaunchKernelGGL(stream_runs_kernel, dim3(workgroups), dim3(256), 0, stream, static_cast<const uint8_t *>(p),
                       lines, runs, sink, 0u);
    return static_cast<int>(hipGetLastError());
}

// `launches` launches of an empty one-wave kernel.
int q4bench_empty(uint32_t launches, hipStream_t stream) {
    for (uint32_t i = 0; i < launches; ++i) hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, stream);
    return static_cast<int>(hipGetLastError());
}

// y[n] = x * rsqrt(mean(x^2) + eps), fp32, one launch.
int q4bench_rms_norm(const float *x, float *y, uint32_t n, float eps, hipStream_t stream) {
    if (x == nullptr || y == nullptr || n == 0) return static_cast<int>(hipErrorInvalidValue);
    hipLaunchKernelGGL(rms_norm_kernel, dim3(1), dim3(kNormThreads), 0, stream, x, y, n, eps);
    return static_cast<int>(hipGetLastError());
}

}  // extern "C"
