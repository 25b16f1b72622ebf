// Row A1: affine unpack + dequant, and the quantized-embedding gather built on it.
//
// One thread owns one 16-byte chunk of packed weights (4 words: 32 values at
// 4 bits, 16 at 8 bits). Every value of a chunk lies in one group because
// group_size >= 32 and chunks are 32/16-value aligned. Reads are 16-byte
// coalesced along a row; the output chunk (64/32 bytes of bf16) is written
// with 16-byte stores.
#include "mi_common.h"

namespace mi {
namespace {

template <typename T, int BITS>
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t *__restrict__ w,
                                                      const T *__restrict__ s,
                                                      const T *__restrict__ b,
                                                      T *__restrict__ out,
                                                      const void *__restrict__ ids, int ids64,
                                                      int64_t rows, int64_t N, int64_t K,
                                                      int gs) {
    constexpr int VPW = 32 / BITS;   // values per word
    constexpr int VPC = 4 * VPW;     // values per 16-byte chunk
    const int64_t cpr = K / VPC;     // chunks per row
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= rows * cpr) return;
    // 32-bit index math (the launcher keeps rows * cpr below 2^31)
    const int64_t r = (unsigned)t / (unsigned)cpr, c = t - r * cpr;
    int64_t n = r;
    if (ids) {
        n = ids64 ? ((const int64_t *)ids)[r] : (int64_t)((const int32_t *)ids)[r];
        n = n < 0 ? 0 : (n >= N ? N - 1 : n);
    }
    const uint4 wv = ld16(w + n * (K / VPW) + c * 4);
    const int64_t k0 = c * VPC;
    const int gsh = __builtin_ctz((unsigned)gs);  // group sizes are powers of two
    const int64_t G = K >> gsh;
    const float sc = (float)s[n * G + (k0 >> gsh)];
    const float bi = (float)b[n * G + (k0 >> gsh)];
    const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
    float v[VPC];
#pragma unroll
    for (int i = 0; i < VPC; ++i) {
        const uint32_t q = (words[i / VPW] >> ((i % VPW) * BITS)) & ((1u << BITS) - 1u);
        v[i] = __builtin_fmaf(sc, (float)q, bi);
    }
    T *o = out + r * K + k0;
    if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int i = 0; i < VPC; i += 4)
            st16(o + i, make_uint4(__float_as_uint(v[i]), __float_as_uint(v[i + 1]),
                                   __float_as_uint(v[i + 2]), __float_as_uint(v[i + 3])));
    } else {
#pragma unroll
        for (int i = 0; i < VPC; i += 8) {
            float f[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) f[j] = v[i + j];
            st16(o + i, pack8<T>(f));
        }
    }
}

template <typename T>
int launch_dequant(const uint32_t *w, const void *s, const void *b, void *out, const void *ids,
                   int ids64, int64_t rows, int64_t N, int64_t K, int gs, int bits,
                   hipStream_t st) {
    const int vpc = bits == 4 ? 32 : 16;
    const int64_t threads = rows * (K / vpc);
    if (threads == 0) return MI_OK;
    if (threads >= ((int64_t)1 << 31))  // the kernel indexes threads in 32 bits
        return fail(MI_ERR_UNSUPPORTED, "dequant of %lld chunks", (long long)threads);
    const dim3 grid((unsigned)ceil_div(threads, 256));
    if (bits == 4)
        dequant_kernel<T, 4><<<grid, 256, 0, st>>>(w, (const T *)s, (const T *)b, (T *)out, ids,
                                                   ids64, rows, N, K, gs);
    else
        dequant_kernel<T, 8><<<grid, 256, 0, st>>>(w, (const T *)s, (const T *)b, (T *)out, ids,
                                                   ids64, rows, N, K, gs);
    return launch_status("affine dequant");
}

int dispatch_dequant(const uint32_t *w, const void *s, const void *b, void *out,
                     const void *ids, int ids64, int64_t rows, int64_t N, int64_t K, int gs,
                     int bits, int dtype, void *stream) {
    if (int e = check_quant(N, K, gs, bits, dtype)) return e;
    if (rows < 0) return fail(MI_ERR_ARG, "negative row count");
    if (!w || !s || !b || (!out && rows)) return fail(MI_ERR_ARG, "null pointer");
    if (!aligned(w, 16) || !aligned(out, 16))
        return fail(MI_ERR_ARG, "packed weights and output must be 16-byte aligned");
    hipStream_t st = as_stream(stream);
    switch (dtype) {
    case MI_BF16: return launch_dequant<bf16>(w, s, b, out, ids, ids64, rows, N, K, gs, bits, st);
    case MI_F16: return launch_dequant<f16>(w, s, b, out, ids, ids64, rows, N, K, gs, bits, st);
    default: return launch_dequant<float>(w, s, b, out, ids, ids64, rows, N, K, gs, bits, st);
    }
}

}  // namespace
}  // namespace mi

extern "C" int mi_affine_dequant(const uint32_t *w, const void *scales, const void *biases,
                                 void *out, int64_t N, int64_t K, int group_size, int bits,
                                 int dtype, void *stream) {
    return mi::dispatch_dequant(w, scales, biases, out, nullptr, 0, N, N, K, group_size, bits,
                                dtype, stream);
}

extern "C" int mi_affine_gather_dequant(const void *ids, int64_t n_ids, int ids_are_64,
                                        const uint32_t *w, const void *scales,
                                        const void *biases, void *out, int64_t N, int64_t K,
                                        int group_size, int bits, int dtype, void *stream) {
    if (!ids && n_ids) return mi::fail(MI_ERR_ARG, "null ids");
    if (N <= 0) return mi::fail(MI_ERR_ARG, "empty embedding table");
    return mi::dispatch_dequant(w, scales, biases, out, ids, ids_are_64 ? 1 : 0, n_ids, N, K,
                                group_size, bits, dtype, stream);
}
