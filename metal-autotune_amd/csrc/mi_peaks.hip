// The device's peaks, measured (include/mi_peaks.h): MFMA issue rate, HBM
// read rate and the launch floor. The reference prices every kernel against
// peaks it microbenchmarks itself (autotuner/measure/peaks.py:1-7, 34-42);
// these kernels are the gfx950 side of that measurement.
#include "mi_common.h"
#include "mi_peaks.h"

namespace mi {
namespace {

constexpr int PEAK_THREADS = 256;

// Four accumulators round-robin: consecutive MFMAs never depend on each other,
// so each wave issues one every 32 cycles when it has the matrix pipe alone.
// The operands are lane-dependent constants (finite, small), the checksum
// folds every accumulator.
__global__ __launch_bounds__(PEAK_THREADS) void peak_mfma_kernel(int iters, float *sink,
                                                                  int64_t *clk) {
    f32x16 acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;
    const unsigned t = threadIdx.x;
    const bf16x8 a = __builtin_bit_cast(bf16x8, (uint4){0x3f803f80u ^ (t & 7u), 0x3f003f00u,
                                                        0x3e803e80u, 0x3f803f80u});
    const bf16x8 b = __builtin_bit_cast(bf16x8, (uint4){0x3c003c00u, 0x3c803c80u ^ (t & 3u),
                                                        0x3d003d00u, 0x3c003c00u});
    const int64_t c0 = (int64_t)__builtin_amdgcn_s_memtime();
    const int64_t r0 = (int64_t)__builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int m = 0; m < 16; ++m)
            acc[m & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[m & 3], 0, 0, 0);
    }
    const int64_t c1 = (int64_t)__builtin_amdgcn_s_memtime();
    const int64_t r1 = (int64_t)__builtin_amdgcn_s_memrealtime();
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) s += acc[i][e];
    const int wave = (int)(blockIdx.x * (PEAK_THREADS / 64) + (t >> 6));
    if ((t & 63) == 0) {
        sink[wave] = s;
        if (clk) {
            clk[2 * wave] = c1 - c0;
            clk[2 * wave + 1] = r1 - r0;
        }
    }
}

// Each workgroup streams one contiguous chunk of the buffer with
// non-temporal 16-byte loads, eight in flight per lane. Measured on MI355X
// over 2 GiB: 7.0-7.1 TB/s, against 6.2 TB/s with ordinary loads and
// 5.4-5.8 TB/s for a grid-stride walk of the same buffer.
constexpr int PEAK_READ_UNROLL = 8;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(PEAK_THREADS) void peak_read_kernel(const uint4 *__restrict__ src,
                                                                  int64_t n16,
                                                                  uint32_t *__restrict__ sink) {
    const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const int64_t b0 = (int64_t)blockIdx.x * per, b1 = b0 + per < n16 ? b0 + per : n16;
    const u32x4 *s = (const u32x4 *)src;
    u32x4 acc = {0u, 0u, 0u, 0u};
    int64_t i = b0 + threadIdx.x;
    for (; i + (PEAK_READ_UNROLL - 1) * PEAK_THREADS < b1; i += PEAK_READ_UNROLL * PEAK_THREADS) {
        u32x4 v[PEAK_READ_UNROLL];
#pragma unroll
        for (int u = 0; u < PEAK_READ_UNROLL; ++u)
            v[u] = __builtin_nontemporal_load(s + i + u * PEAK_THREADS);
#pragma unroll
        for (int u = 0; u < PEAK_READ_UNROLL; ++u) acc ^= v[u];
    }
    // the tail as one predicated batch: every load is issued before the first
    // is used, also when a workgroup's chunk is only a few loads per lane
    // (small buffers over many workgroups)
    if (i < b1) {
        u32x4 v[PEAK_READ_UNROLL];
#pragma unroll
        for (int u = 0; u < PEAK_READ_UNROLL; ++u) {
            const int64_t k = i + u * PEAK_THREADS;
            v[u] = k < b1 ? __builtin_nontemporal_load(s + k) : (u32x4){0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < PEAK_READ_UNROLL; ++u) acc ^= v[u];
    }
    uint32_t a = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
    // one word per workgroup: lanes fold by shuffle, waves through LDS
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) a ^= (uint32_t)__shfl_xor((int)a, o, 64);
    __shared__ uint32_t part[PEAK_THREADS / 64];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = a;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t r = 0;
        for (int w = 0; w < PEAK_THREADS / 64; ++w) r ^= part[w];
        sink[blockIdx.x] = r;
    }
}

__global__ void peak_empty_kernel() {}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int mi_peak_mfma_bf16(int blocks, int iters, float *sink, int64_t *clk, void *stream) {
    if (blocks <= 0 || iters <= 0 || !sink) return fail(MI_ERR_ARG, "peak_mfma: blocks, iters, sink");
    peak_mfma_kernel<<<blocks, PEAK_THREADS, 0, as_stream(stream)>>>(iters, sink, clk);
    return launch_status("peak_mfma");
}

extern "C" int mi_peak_read(const void *src, int64_t bytes, int blocks, uint32_t *sink,
                            void *stream) {
    if (!src || !sink || blocks <= 0 || bytes <= 0 || bytes % 64 || !aligned(src, 16))
        return fail(MI_ERR_ARG, "peak_read: src 16-byte aligned, bytes a positive multiple of 64");
    peak_read_kernel<<<blocks, PEAK_THREADS, 0, as_stream(stream)>>>((const uint4 *)src, bytes / 16,
                                                                     sink);
    return launch_status("peak_read");
}

extern "C" int mi_peak_empty(void *stream) {
    peak_empty_kernel<<<1, 64, 0, as_stream(stream)>>>();
    return launch_status("peak_empty");
}
