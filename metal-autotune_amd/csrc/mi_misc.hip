// Rows A8 (SwiGLU), A9 (LFM2 short-conv core), A10 (fp32 linear + exact GELU
// for the tiny-MLP region) and the greedy-argmax glue of A12. All HBM- or
// launch-bound elementwise/row work: 16-byte vector loads where the layout
// allows, one thread per 8 values.
#include <math.h>

#include <mutex>

#include "mi_common.h"

namespace mi {
namespace {

template <typename T> __device__ __forceinline__ float swiglu_one(float g, float u) {
    const float sig = (float)cvt<T>(1.0f / (1.0f + __expf(-g)));
    const float act = (float)cvt<T>(g * sig);
    return act * u;
}

template <typename T>
__global__ __launch_bounds__(256) void swiglu_kernel(const T *__restrict__ g,
                                                     const T *__restrict__ u, T *__restrict__ y,
                                                     int64_t n, int vec_ok) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if constexpr (sizeof(T) == 2) {
        if (vec_ok) {
            if (t * 8 >= n) return;
            float gf[8], uf[8];
            unpack8<T>(ld16(g + 8 * t), gf);
            unpack8<T>(ld16(u + 8 * t), uf);
#pragma unroll
            for (int i = 0; i < 8; ++i) gf[i] = swiglu_one<T>(gf[i], uf[i]);
            st16(y + 8 * t, pack8<T>(gf));
            return;
        }
    }
    for (int64_t i = t * 8; i < n && i < t * 8 + 8; ++i)
        y[i] = cvt<T>(swiglu_one<T>((float)g[i], (float)u[i]));
}

// Grid rows 0..L-1 produce out; rows L, L+1 copy the last two padded rows into
// state_out. pad[i] = state_in[i] (or 0) for i < 2, bx[i-2] otherwise.
// VEC (D a multiple of 8, every pointer 16-byte aligned): a thread's 8
// channels move as 16-byte loads and stores -- the three taps of bx, c, the
// 24 weights (w is [D, 3], so 8 channels' weights are 48 contiguous bytes),
// the state rows -- with the same per-channel arithmetic as the scalar path.
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void shortconv_kernel(const T *__restrict__ bx,
                                                        const T *__restrict__ c,
                                                        const T *__restrict__ w,
                                                        const T *__restrict__ st_in,
                                                        T *__restrict__ out,
                                                        T *__restrict__ st_out, int64_t B,
                                                        int64_t L, int64_t D) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t dchunks = ceil_div(D, 8);
    if (t >= B * (L + 2) * dchunks) return;
    // 32-bit index math (the launcher keeps the thread count below 2^31)
    const unsigned ut = (unsigned)t, udc = (unsigned)dchunks, ulr = (unsigned)(L + 2);
    const int64_t dc = ut % udc, row = (ut / udc) % ulr, b = ut / (udc * ulr);
    if constexpr (VEC && sizeof(T) == 2) {
        const int64_t d0 = dc * 8;
        auto padv = [&](int64_t i, float (&f)[8]) {
            if (i >= 2) {
                unpack8<T>(ld16(bx + (b * L + i - 2) * D + d0), f);
            } else if (st_in) {
                unpack8<T>(ld16(st_in + (b * 2 + i) * D + d0), f);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) f[e] = 0.0f;
            }
        };
        if (row < L) {
            float p0[8], p1[8], p2[8], cf[8], wf[24];
            padv(row, p0);
            padv(row + 1, p1);
            padv(row + 2, p2);
            unpack8<T>(ld16(c + (b * L + row) * D + d0), cf);
#pragma unroll
            for (int j = 0; j < 3; ++j) {
                float tmp[8];
                unpack8<T>(ld16(w + d0 * 3 + 8 * j), tmp);
#pragma unroll
                for (int e = 0; e < 8; ++e) wf[8 * j + e] = tmp[e];
            }
            float o[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float acc = p0[e] * wf[3 * e + 0];
                acc = __builtin_fmaf(p1[e], wf[3 * e + 1], acc);
                acc = __builtin_fmaf(p2[e], wf[3 * e + 2], acc);
                const float conv = (float)cvt<T>(acc);
                o[e] = cf[e] * conv;
            }
            st16(out + (b * L + row) * D + d0, pack8<T>(o));
        } else if (st_out) {
            const int64_t i = row - L;  // 0 or 1
            float f[8];
            padv(L + i, f);
            st16(st_out + (b * 2 + i) * D + d0, pack8<T>(f));
        }
        return;
    }
    auto pad = [&](int64_t i, int64_t d) -> float {
        if (i >= 2) return (float)bx[(b * L + i - 2) * D + d];
        return st_in ? (float)st_in[(b * 2 + i) * D + d] : 0.0f;
    };
    for (int64_t d = dc * 8; d < D && d < dc * 8 + 8; ++d) {
        if (row < L) {
            float acc = pad(row, d) * (float)w[d * 3 + 0];
            acc = __builtin_fmaf(pad(row + 1, d), (float)w[d * 3 + 1], acc);
            acc = __builtin_fmaf(pad(row + 2, d), (float)w[d * 3 + 2], acc);
            const float conv = (float)cvt<T>(acc);
            out[(b * L + row) * D + d] = cvt<T>((float)c[(b * L + row) * D + d] * conv);
        } else if (st_out) {
            const int64_t i = row - L;  // 0 or 1
            st_out[(b * 2 + i) * D + d] = cvt<T>(pad(L + i, d));
        }
    }
}

// fp32 linear: 16x16 output tile per 256-thread block, K in 16-wide LDS tiles,
// each output's sum sequential in k.
__global__ __launch_bounds__(256) void linear_f32_kernel(const float *__restrict__ x,
                                                         const float *__restrict__ w,
                                                         const float *__restrict__ bias,
                                                         float *__restrict__ y, int64_t M,
                                                         int64_t N, int64_t K, int act) {
    __shared__ float xs[16][17];
    __shared__ float ws[16][17];
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    const int64_t n = (int64_t)blockIdx.x * 16 + tx;
    const int64_t m = (int64_t)blockIdx.y * 16 + ty;
    float acc = 0.0f;
    for (int64_t k0 = 0; k0 < K; k0 += 16) {
        const int64_t xm = (int64_t)blockIdx.y * 16 + ty, wn = (int64_t)blockIdx.x * 16 + ty;
        xs[ty][tx] = (xm < M && k0 + tx < K) ? x[xm * K + k0 + tx] : 0.0f;
        ws[ty][tx] = (wn < N && k0 + tx < K) ? w[wn * K + k0 + tx] : 0.0f;
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 16; ++kk) acc = __builtin_fmaf(xs[ty][kk], ws[tx][kk], acc);
        __syncthreads();
    }
    if (m >= M || n >= N) return;
    if (bias) acc += bias[n];
    if (act == MI_ACT_GELU) acc = acc * (1.0f + erff(acc / 1.41421356237f)) / 2.0f;
    y[m * N + n] = acc;
}

// Config 1's whole MLP in one launch: y = gelu(x W1^T + b1) W2^T + b2, fp32.
// Workgroup (c, rb) takes hidden units [64 c, 64 c + 64) for token rows
// [8 rb, 8 rb + 8): phase 1 computes those gelu(h) values into LDS (each a
// sequential fma chain over k, plus b1); phase 2 multiplies them into a
// partial y tile [8, N] over its 64 hidden units and stores it in the
// workspace. The last workgroup of a row block to finish (a ticket counter
// per row block) adds the partials of chunks 0, 1, 2, ... in that fixed order,
// then b2, and writes y, so the result does not depend on which workgroup
// finished last. It then resets the counter: the workspace's counters are zero
// before the first call and after every call.
constexpr int MLP_HT = 64;      // hidden units per workgroup
constexpr int MLP_RT = 8;       // token rows per workgroup
constexpr int MLP_THREADS = 256;
constexpr int64_t MLP_MAX_K = 1024;  // x rows staged in LDS: 8 x 1024 fp32 = 32 KB

__device__ __forceinline__ float gelu_erf(float v) {
    return v * (1.0f + erff(v / 1.41421356237f)) / 2.0f;
}

__global__ __launch_bounds__(MLP_THREADS) void gelu_mlp_f32_kernel(
    const float *__restrict__ x, const float *__restrict__ w1, const float *__restrict__ b1,
    const float *__restrict__ w2, const float *__restrict__ b2, float *__restrict__ y,
    float *__restrict__ part, unsigned *__restrict__ tickets, int64_t M, int64_t K, int64_t H,
    int64_t N) {
    extern __shared__ __attribute__((aligned(16))) float mlp_lds[];
    float *xs = mlp_lds;                       // [MLP_RT][K]
    float *hs = mlp_lds + MLP_RT * K;          // [MLP_RT][MLP_HT]
    __shared__ int last;
    const int t = threadIdx.x;
    const int64_t c = blockIdx.x, rb = blockIdx.y;
    const int64_t C = gridDim.x;
    const int64_t r0 = rb * MLP_RT;
    const int rows = (int)(M - r0 < MLP_RT ? M - r0 : MLP_RT);

    // stage the row block of x (rows past M read as zero)
    for (int64_t i = t; i < MLP_RT * K / 4; i += MLP_THREADS) {
        const int64_t r = (4 * i) / K, k = 4 * i - r * K;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < rows) v = *(const float4 *)(x + (r0 + r) * K + k);
        *(float4 *)(xs + r * K + k) = v;
    }
    __syncthreads();

    // phase 1: lane j of wave w computes hidden unit 64 c + j for rows w, w + 4
    {
        const int j = t & 63, w = t >> 6;
        const int64_t hj = c * MLP_HT + j;
        const int64_t hrow = hj < H ? hj : H - 1;  // clamped, valid row
        const float *wr = w1 + hrow * K;
        float a0 = 0.0f, a1 = 0.0f;
        for (int64_t k = 0; k < K; k += 4) {
            const float4 wv = *(const float4 *)(wr + k);
            const float4 xa = *(const float4 *)(xs + w * K + k);
            const float4 xb = *(const float4 *)(xs + (w + 4) * K + k);
            a0 = __builtin_fmaf(xa.x, wv.x, a0);
            a0 = __builtin_fmaf(xa.y, wv.y, a0);
            a0 = __builtin_fmaf(xa.z, wv.z, a0);
            a0 = __builtin_fmaf(xa.w, wv.w, a0);
            a1 = __builtin_fmaf(xb.x, wv.x, a1);
            a1 = __builtin_fmaf(xb.y, wv.y, a1);
            a1 = __builtin_fmaf(xb.z, wv.z, a1);
            a1 = __builtin_fmaf(xb.w, wv.w, a1);
        }
        const float bias = b1 ? b1[hrow] : 0.0f;
        hs[w * MLP_HT + j] = hj < H ? gelu_erf(a0 + bias) : 0.0f;
        hs[(w + 4) * MLP_HT + j] = hj < H ? gelu_erf(a1 + bias) : 0.0f;
    }
    __syncthreads();

    // phase 2: thread t takes output columns n = t, t + 256, ... for all rows
    const int64_t hbase = c * MLP_HT;
    const int hn = (int)(H - hbase < MLP_HT ? H - hbase : MLP_HT);  // a multiple of 4
    float *pc = part + c * (M * N);
    for (int64_t n = t; n < N; n += MLP_THREADS) {
        const float *wr = w2 + n * H + hbase;
        float acc[MLP_RT];
#pragma unroll
        for (int r = 0; r < MLP_RT; ++r) acc[r] = 0.0f;
        for (int hh = 0; hh < hn; hh += 4) {
            const float4 wv = *(const float4 *)(wr + hh);
#pragma unroll
            for (int r = 0; r < MLP_RT; ++r) {
                const float4 hv = *(const float4 *)(hs + r * MLP_HT + hh);
                acc[r] = __builtin_fmaf(hv.x, wv.x, acc[r]);
                acc[r] = __builtin_fmaf(hv.y, wv.y, acc[r]);
                acc[r] = __builtin_fmaf(hv.z, wv.z, acc[r]);
                acc[r] = __builtin_fmaf(hv.w, wv.w, acc[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < MLP_RT; ++r)
            if (r < rows) pc[(r0 + r) * N + n] = acc[r];
    }

    // phase 3: the last workgroup of this row block reduces the partials
    __threadfence();  // release: this workgroup's partials before its ticket
    __syncthreads();
    if (t == 0) {
        const unsigned ticket = atomicAdd(&tickets[rb], 1u);
        last = ticket == (unsigned)(C - 1);
    }
    __syncthreads();
    if (!last) return;
    __threadfence();  // acquire: every partial of the row block is visible
    for (int64_t i = t; i < (int64_t)rows * N; i += MLP_THREADS) {
        const int64_t r = i / N, n = i - r * N;
        const int64_t o = (r0 + r) * N + n;
        float s = part[o];
        for (int64_t cc = 1; cc < C; ++cc) s += part[cc * (M * N) + o];
        if (b2) s += b2[n];
        y[o] = s;
    }
    if (t == 0) __hip_atomic_store(&tickets[rb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Greedy argmax: one 1024-thread workgroup per row. Each thread keeps the
// first maximum of the elements it scans (in increasing index order); the
// (value, index) pairs are then combined with the lowest index winning a tie.
// NaN never wins (every comparison with it is false); a row with no non-NaN
// value gives 0. VEC: the row is read in 16-byte chunks, 8 chunks in flight
// per thread (rows must be 16-byte aligned and V a multiple of the chunk).
constexpr int AM_THREADS = 1024;
constexpr int AM_BATCH = 8;

__device__ __forceinline__ void am_take(float v, int64_t i, float &best, int64_t &bi) {
    if (v > best || (bi < 0 && !isnan(v))) {
        best = v;
        bi = i;
    }
}

__device__ __forceinline__ void am_merge(float ov, int64_t oi, float &best, int64_t &bi) {
    if (oi >= 0 && (bi < 0 || ov > best || (ov == best && oi < bi))) {
        best = ov;
        bi = oi;
    }
}

template <typename T, bool VEC>
__global__ __launch_bounds__(AM_THREADS) void argmax_kernel(const T *__restrict__ x,
                                                            int32_t *__restrict__ out, int64_t V) {
    constexpr int E = 16 / (int)sizeof(T);  // values per 16-byte chunk
    constexpr int NW = AM_THREADS / 64;
    __shared__ float sv[NW];
    __shared__ int64_t si[NW];
    const T *row = x + (int64_t)blockIdx.x * V;
    float best = -INFINITY;
    int64_t bi = -1;
    if constexpr (VEC) {
        const int64_t nc = V / E;
        for (int64_t c0 = threadIdx.x; c0 < nc; c0 += (int64_t)AM_THREADS * AM_BATCH) {
            uint4 d[AM_BATCH];
#pragma unroll
            for (int u = 0; u < AM_BATCH; ++u) {
                const int64_t c = c0 + (int64_t)u * AM_THREADS;
                d[u] = ld16(row + (c < nc ? c : nc - 1) * E);  // clamped: always in bounds
            }
#pragma unroll
            for (int u = 0; u < AM_BATCH; ++u) {
                const int64_t c = c0 + (int64_t)u * AM_THREADS;
                if (c >= nc) break;
                float f[E];
                if constexpr (sizeof(T) == 2) {
                    unpack8<T>(d[u], f);
                } else {
                    f[0] = __uint_as_float(d[u].x);
                    f[1] = __uint_as_float(d[u].y);
                    f[2] = __uint_as_float(d[u].z);
                    f[3] = __uint_as_float(d[u].w);
                }
#pragma unroll
                for (int e = 0; e < E; ++e) am_take(f[e], c * E + e, best, bi);
            }
        }
    } else {
        for (int64_t i = threadIdx.x; i < V; i += AM_THREADS) am_take((float)row[i], i, best, bi);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const int64_t oi = __shfl_xor(bi, o, 64);
        am_merge(ov, oi, best, bi);
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sv[wave] = best;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w2 = 1; w2 < NW; ++w2) am_merge(sv[w2], si[w2], best, bi);
        out[blockIdx.x] = (int32_t)(bi < 0 ? 0 : bi);
    }
}

// Split argmax: a row is cut into spans of AM_SPAN units (16-byte chunks when
// VEC, else single values); workgroup (g, row) reduces span g to one
// (value, index) partial, then one wave per row merges the row's partials.
// The merge is a total order (larger value, then lower index; NaN never
// wins), so the result equals the one-workgroup kernel's.
constexpr int AM_SPLIT_THREADS = 256;
constexpr int AM_SPAN_CHUNKS = 2 * AM_SPLIT_THREADS;  // 16-byte chunks per workgroup
constexpr int AM_SPAN_VALUES = 8 * AM_SPLIT_THREADS;  // values per workgroup (scalar path)

struct AmPart {
    float v;
    int32_t i;  // -1: the span holds no non-NaN value
};

template <typename T, bool VEC>
__global__ __launch_bounds__(AM_SPLIT_THREADS) void argmax_part_kernel(const T *__restrict__ x,
                                                                        AmPart *__restrict__ part,
                                                                        int64_t V) {
    constexpr int E = 16 / (int)sizeof(T);
    constexpr int NW = AM_SPLIT_THREADS / 64;
    __shared__ float sv[NW];
    __shared__ int32_t si[NW];
    const T *row = x + (int64_t)blockIdx.y * V;
    float best = -INFINITY;
    int64_t bi = -1;
    if constexpr (VEC) {
        const int64_t nc = V / E;
        const int64_t c0 = (int64_t)blockIdx.x * AM_SPAN_CHUNKS + threadIdx.x;
        uint4 d[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int64_t c = c0 + u * AM_SPLIT_THREADS;
            d[u] = ld16(row + (c < nc ? c : nc - 1) * E);  // clamped: always in bounds
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int64_t c = c0 + u * AM_SPLIT_THREADS;
            if (c >= nc) break;
            float f[E];
            if constexpr (sizeof(T) == 2) {
                unpack8<T>(d[u], f);
            } else {
                f[0] = __uint_as_float(d[u].x);
                f[1] = __uint_as_float(d[u].y);
                f[2] = __uint_as_float(d[u].z);
                f[3] = __uint_as_float(d[u].w);
            }
#pragma unroll
            for (int e = 0; e < E; ++e) am_take(f[e], c * E + e, best, bi);
        }
    } else {
        const int64_t i0 = (int64_t)blockIdx.x * AM_SPAN_VALUES;
        const int64_t i1 = i0 + AM_SPAN_VALUES < V ? i0 + AM_SPAN_VALUES : V;
        for (int64_t i = i0 + threadIdx.x; i < i1; i += AM_SPLIT_THREADS)
            am_take((float)row[i], i, best, bi);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const int64_t oi = __shfl_xor(bi, o, 64);
        am_merge(ov, oi, best, bi);
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sv[wave] = best;
        si[wave] = (int32_t)bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w2 = 1; w2 < NW; ++w2) am_merge(sv[w2], si[w2], best, bi);
        part[(int64_t)blockIdx.y * gridDim.x + blockIdx.x] = AmPart{best, (int32_t)bi};
    }
}

__global__ __launch_bounds__(64) void argmax_merge_kernel(const AmPart *__restrict__ part, int G,
                                                          int32_t *__restrict__ out) {
    const AmPart *p = part + (int64_t)blockIdx.x * G;
    float best = -INFINITY;
    int64_t bi = -1;
    for (int g = threadIdx.x; g < G; g += 64) am_merge(p[g].v, p[g].i, best, bi);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const int64_t oi = __shfl_xor(bi, o, 64);
        am_merge(ov, oi, best, bi);
    }
    if (threadIdx.x == 0) out[blockIdx.x] = (int32_t)(bi < 0 ? 0 : bi);
}

// spans per row of the split argmax
int64_t am_spans(int64_t V, int esize, bool vec) {
    return vec ? ceil_div(V * esize / 16, AM_SPAN_CHUNKS) : ceil_div(V, AM_SPAN_VALUES);
}

}  // namespace
}  // namespace mi

// Scratch of mi_argmax_noalloc: the per-span partials of the split argmax,
// AM_NOALLOC_PARTS entries (64 KiB) in a file-scope device array, one copy per
// GPU, held until the process ends. Host code never passes the array's name
// to a kernel (on the host it is only a stand-in symbol): the first call on a
// device looks up that device's copy with hipGetSymbolAddress and keeps the
// pointer. Calls on one GPU share the array, so calls that overlap on one GPU
// race; every call overwrites the partials it reads, so nothing has to start
// at zero.
#define AM_NOALLOC_PARTS 8192
static __device__ __align__(256) mi::AmPart scratch[AM_NOALLOC_PARTS];

namespace {
constexpr int AM_MAX_DEVICES = 64;
std::mutex am_scratch_lock;
mi::AmPart *am_scratch_ptr[AM_MAX_DEVICES];

// This device's copy of `scratch` (found once per device), or NULL after
// recording an error.
mi::AmPart *am_scratch(int dev) {
    if (dev < 0 || dev >= AM_MAX_DEVICES) {
        mi::fail(MI_ERR_ARG, "argmax_noalloc: device %d beyond %d", dev, AM_MAX_DEVICES);
        return nullptr;
    }
    std::lock_guard<std::mutex> guard(am_scratch_lock);
    if (am_scratch_ptr[dev] == nullptr) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            mi::fail(MI_ERR_LAUNCH, "argmax_noalloc: hipGetSymbolAddress on device %d: %s", dev,
                     hipGetErrorString(e));
            return nullptr;
        }
        am_scratch_ptr[dev] = (mi::AmPart *)p;
    }
    return am_scratch_ptr[dev];
}
}  // namespace

using namespace mi;

extern "C" int mi_swiglu(const void *g, const void *u, void *y, int64_t n, int dtype,
                         void *stream) {
    if (!valid_dtype(dtype)) return fail(MI_ERR_UNSUPPORTED, "dtype code %d", dtype);
    if (n < 0) return fail(MI_ERR_ARG, "negative size");
    if (n == 0) return MI_OK;
    if (!g || !u || !y) return fail(MI_ERR_ARG, "null pointer");
    hipStream_t st = as_stream(stream);
    const unsigned grid = (unsigned)ceil_div(ceil_div(n, 8), 256);
    const int vec = n % 8 == 0 && aligned(g, 16) && aligned(u, 16) && aligned(y, 16);
    if (dtype == MI_BF16)
        swiglu_kernel<bf16><<<grid, 256, 0, st>>>((const bf16 *)g, (const bf16 *)u, (bf16 *)y, n,
                                                  vec);
    else if (dtype == MI_F16)
        swiglu_kernel<f16><<<grid, 256, 0, st>>>((const f16 *)g, (const f16 *)u, (f16 *)y, n,
                                                 vec);
    else
        swiglu_kernel<float><<<grid, 256, 0, st>>>((const float *)g, (const float *)u,
                                                    (float *)y, n, vec);
    return launch_status("swiglu");
}

extern "C" int mi_shortconv(const void *bx, const void *c, const void *w, const void *state_in,
                            void *out, void *state_out, int64_t B, int64_t L, int64_t D,
                            int dtype, void *stream) {
    if (!valid_dtype(dtype)) return fail(MI_ERR_UNSUPPORTED, "dtype code %d", dtype);
    if (B < 0 || L < 0 || D <= 0) return fail(MI_ERR_ARG, "shortconv shape");
    if (state_out && (state_out == state_in || state_out == bx || state_out == c))
        return fail(MI_ERR_ARG, "state_out must not alias an input");
    if (B * L && (!bx || !c || !w || !out)) return fail(MI_ERR_ARG, "null pointer");
    const int64_t threads = B * (L + 2) * ceil_div(D, 8);
    if (threads == 0) return MI_OK;
    if (threads >= ((int64_t)1 << 31))  // the kernel indexes threads in 32 bits
        return fail(MI_ERR_UNSUPPORTED, "shortconv of %lld 8-channel chunks", (long long)threads);
    hipStream_t st = as_stream(stream);
    const unsigned grid = (unsigned)ceil_div(threads, 256);
    const bool vec = D % 8 == 0 && aligned(bx, 16) && aligned(c, 16) && aligned(w, 16) &&
                     aligned(out, 16) && (!state_in || aligned(state_in, 16)) &&
                     (!state_out || aligned(state_out, 16));
#define MI_SC(TT)                                                                               \
    do {                                                                                        \
        if (vec)                                                                                \
            shortconv_kernel<TT, true><<<grid, 256, 0, st>>>(                                   \
                (const TT *)bx, (const TT *)c, (const TT *)w, (const TT *)state_in, (TT *)out,  \
                (TT *)state_out, B, L, D);                                                      \
        else                                                                                    \
            shortconv_kernel<TT, false><<<grid, 256, 0, st>>>(                                  \
                (const TT *)bx, (const TT *)c, (const TT *)w, (const TT *)state_in, (TT *)out,  \
                (TT *)state_out, B, L, D);                                                      \
    } while (0)
    if (dtype == MI_BF16)
        MI_SC(bf16);
    else if (dtype == MI_F16)
        MI_SC(f16);
    else
        MI_SC(float);
#undef MI_SC
    return launch_status("shortconv");
}

extern "C" int mi_linear_f32(const float *x, const float *w, const float *bias, float *y,
                             int64_t M, int64_t N, int64_t K, int act, void *stream) {
    if (M < 0 || N < 0 || K <= 0) return fail(MI_ERR_ARG, "linear shape");
    if (act != MI_ACT_NONE && act != MI_ACT_GELU)
        return fail(MI_ERR_UNSUPPORTED, "linear activation %d", act);
    if (M == 0 || N == 0) return MI_OK;
    if (!x || !w || !y) return fail(MI_ERR_ARG, "null pointer");
    const dim3 grid((unsigned)ceil_div(N, 16), (unsigned)ceil_div(M, 16));
    linear_f32_kernel<<<grid, 256, 0, as_stream(stream)>>>(x, w, bias, y, M, N, K, act);
    return launch_status("linear_f32");
}

// Workspace of mi_gelu_mlp_f32: one ticket counter per row block, then the
// partial y tiles of every hidden chunk, 256-byte aligned.
// The per-row-block ticket counters take a fixed prefix sized for the largest
// grid (65535 row blocks), whatever M is: a workspace reused across calls of
// different M then never has one call's partial sums over another call's
// counters (a prefix sized by M let a smaller call's partials land where a
// larger call reads its counters).
constexpr int64_t MLP_MAX_ROW_BLOCKS = 65535;
static int64_t mlp_tickets_bytes() { return ceil_div(MLP_MAX_ROW_BLOCKS * 4, 256) * 256; }

extern "C" int64_t mi_gelu_mlp_f32_workspace_bytes(int64_t M, int64_t K, int64_t H, int64_t N) {
    (void)K;
    if (M <= 0 || H <= 0 || N <= 0) return 0;
    return mlp_tickets_bytes() + ceil_div(H, MLP_HT) * M * N * (int64_t)sizeof(float);
}

extern "C" int mi_gelu_mlp_f32(const float *x, const float *w1, const float *b1, const float *w2,
                               const float *b2, float *y, int64_t M, int64_t K, int64_t H,
                               int64_t N, void *workspace, int64_t workspace_bytes,
                               void *stream) {
    if (M < 0 || K <= 0 || H <= 0 || N < 0) return fail(MI_ERR_ARG, "gelu mlp shape");
    if (K % 4 || H % 4)
        return fail(MI_ERR_UNSUPPORTED, "gelu mlp needs K and H multiples of 4 (K=%lld H=%lld)",
                    (long long)K, (long long)H);
    if (K > MLP_MAX_K) return fail(MI_ERR_UNSUPPORTED, "gelu mlp K=%lld above %lld", (long long)K,
                                   (long long)MLP_MAX_K);
    if (M == 0 || N == 0) return MI_OK;
    if (!x || !w1 || !w2 || !y || !workspace) return fail(MI_ERR_ARG, "null pointer");
    if (!aligned(x, 16) || !aligned(w1, 16) || !aligned(w2, 16) || !aligned(workspace, 256))
        return fail(MI_ERR_ARG, "gelu mlp: x, w1, w2 16-byte aligned, workspace 256-byte aligned");
    if (ceil_div(M, MLP_RT) > MLP_MAX_ROW_BLOCKS) return fail(MI_ERR_ARG, "gelu mlp: too many rows");
    const int64_t need = mi_gelu_mlp_f32_workspace_bytes(M, K, H, N);
    if (workspace_bytes < need)
        return fail(MI_ERR_ARG, "gelu mlp workspace of %lld bytes, %lld needed",
                    (long long)workspace_bytes, (long long)need);
    unsigned *tickets = (unsigned *)workspace;
    float *part = (float *)((char *)workspace + mlp_tickets_bytes());
    const dim3 grid((unsigned)ceil_div(H, MLP_HT), (unsigned)ceil_div(M, MLP_RT));
    const size_t lds = (size_t)(MLP_RT * K + MLP_RT * MLP_HT) * sizeof(float);
    gelu_mlp_f32_kernel<<<grid, MLP_THREADS, lds, as_stream(stream)>>>(x, w1, b1, w2, b2, y, part,
                                                                       tickets, M, K, H, N);
    return launch_status("gelu mlp");
}

extern "C" int64_t mi_argmax_workspace_bytes(int64_t rows, int64_t V) {
    if (rows <= 0 || V <= 0) return 0;
    return rows * ceil_div(V, AM_SPAN_VALUES) * (int64_t)sizeof(AmPart);
}

extern "C" int mi_argmax(const void *x, int32_t *out, int64_t rows, int64_t V, int dtype,
                         void *workspace, int64_t workspace_bytes, void *stream) {
    if (!valid_dtype(dtype)) return fail(MI_ERR_UNSUPPORTED, "dtype code %d", dtype);
    if (rows < 0 || V <= 0) return fail(MI_ERR_ARG, "argmax shape");
    if (V > INT32_MAX) return fail(MI_ERR_ARG, "argmax row of %lld values exceeds int32", (long long)V);
    if (rows == 0) return MI_OK;
    if (!x || !out) return fail(MI_ERR_ARG, "null pointer");
    if (workspace && workspace_bytes < mi_argmax_workspace_bytes(rows, V))
        return fail(MI_ERR_ARG, "argmax workspace of %lld bytes, %lld needed",
                    (long long)workspace_bytes, (long long)mi_argmax_workspace_bytes(rows, V));
    if (workspace && !aligned(workspace, 8)) return fail(MI_ERR_ARG, "argmax workspace alignment");
    if (workspace && rows > 65535) return fail(MI_ERR_ARG, "argmax: more than 65535 rows");
    hipStream_t st = as_stream(stream);
    const int esize = dtype == MI_F32 ? 4 : 2;
    const bool vec = aligned(x, 16) && (V * esize) % 16 == 0;
    const int64_t G = am_spans(V, esize, vec);
    AmPart *part = (AmPart *)workspace;
#define MI_AM(TT)                                                                               \
    do {                                                                                        \
        if (part) {                                                                             \
            const dim3 grid((unsigned)G, (unsigned)rows);                                       \
            if (vec)                                                                            \
                argmax_part_kernel<TT, true><<<grid, AM_SPLIT_THREADS, 0, st>>>((const TT *)x,  \
                                                                               part, V);       \
            else                                                                                \
                argmax_part_kernel<TT, false><<<grid, AM_SPLIT_THREADS, 0, st>>>((const TT *)x, \
                                                                                part, V);      \
            argmax_merge_kernel<<<(unsigned)rows, 64, 0, st>>>(part, (int)G, out);             \
        } else if (vec) {                                                                       \
            argmax_kernel<TT, true><<<(unsigned)rows, AM_THREADS, 0, st>>>((const TT *)x, out, V); \
        } else {                                                                                \
            argmax_kernel<TT, false><<<(unsigned)rows, AM_THREADS, 0, st>>>((const TT *)x, out, V); \
        }                                                                                       \
    } while (0)
    if (dtype == MI_BF16)
        MI_AM(bf16);
    else if (dtype == MI_F16)
        MI_AM(f16);
    else
        MI_AM(float);
#undef MI_AM
    return launch_status("argmax");
}

extern "C" int mi_argmax_noalloc(const void *x, int32_t *out, int64_t rows, int64_t V, int dtype,
                                 void *stream) {
    if (!valid_dtype(dtype)) return fail(MI_ERR_UNSUPPORTED, "dtype code %d", dtype);
    if (rows < 0 || V <= 0) return fail(MI_ERR_ARG, "argmax shape");
    if (V > INT32_MAX) return fail(MI_ERR_ARG, "argmax row of %lld values exceeds int32", (long long)V);
    if (rows == 0) return MI_OK;
    if (!x || !out) return fail(MI_ERR_ARG, "null pointer");
    const int esize = dtype == MI_F32 ? 4 : 2;
    const bool vec = aligned(x, 16) && (V * esize) % 16 == 0;
    const int64_t G = am_spans(V, esize, vec);
    if (rows > 65535 || rows * G > AM_NOALLOC_PARTS)
        return fail(MI_ERR_ARG,
                    "argmax_noalloc: %lld rows x %lld spans of partials exceed its fixed scratch "
                    "of %d (use mi_argmax with a workspace)",
                    (long long)rows, (long long)G, AM_NOALLOC_PARTS);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(MI_ERR_LAUNCH, "argmax_noalloc: no device");
    AmPart *part = am_scratch(dev);
    if (!part) return MI_ERR_LAUNCH;
    hipStream_t st = as_stream(stream);
    const dim3 grid((unsigned)G, (unsigned)rows);
#define MI_AMN(TT)                                                                              \
    do {                                                                                        \
        if (vec)                                                                                \
            argmax_part_kernel<TT, true><<<grid, AM_SPLIT_THREADS, 0, st>>>((const TT *)x, part, \
                                                                           V);                 \
        else                                                                                    \
            argmax_part_kernel<TT, false><<<grid, AM_SPLIT_THREADS, 0, st>>>((const TT *)x,     \
                                                                            part, V);          \
        argmax_merge_kernel<<<(unsigned)rows, 64, 0, st>>>(part, (int)G, out);                 \
    } while (0)
    if (dtype == MI_BF16)
        MI_AMN(bf16);
    else if (dtype == MI_F16)
        MI_AMN(f16);
    else
        MI_AMN(float);
#undef MI_AMN
    return launch_status("argmax_noalloc");
}
