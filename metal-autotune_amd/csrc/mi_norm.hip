// Rows A5 (RMSNorm, and the [qmm, add, rms_norm] region) and A6 (q/k-norm + RoPE).
//
// Both are HBM/launch-bound single-pass wave reductions: one wave (or a
// power-of-two lane group) owns a row, sums squares in fp32 with an xor-shuffle
// tree, and writes T(w * T(x * inv)) -- the two-rounding form the reference's
// exact-verified LFM2 norm stage uses (prefill_bk64.stages/1.metal:34-42).
#include <math.h>

#include "mi_common.h"

namespace mi {
int qmm_residual_launch(const void *x, const uint32_t *w, const void *s, const void *b,
                        const void *resid, void *y, int64_t M, int64_t N, int64_t K, int gs,
                        int bits, int dtype, void *stream);
int64_t qmm_parts_bytes(int64_t M, int64_t N, int64_t K, int gs, int bits, int dtype);
int qmm_parts_launch(const void *x, const uint32_t *w, const void *s, const void *b, float *part,
                     int64_t M, int64_t N, int64_t K, int gs, int bits, int dtype, void *stream);

namespace {

// The sum over a wave, the same value in every lane: pairs within quads, then
// quad sums across a half-row (mirror), half-row sums across a row (mirror),
// all through DPP (no LDS round trip; the xor-shuffle tree took six
// ds_bpermute instructions, each a dependent trip through the LDS unit), then
// ((row 0 + row 1) + (row 2 + row 3)) from the four rows' lane 0. Every step
// adds two values that every lane of the group holds alike, so all lanes end
// with the same bits.
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (r0 + r1) + (r2 + r3);
}

template <typename T>
__global__ __launch_bounds__(256) void rms_kernel(const T *__restrict__ x, const T *__restrict__ w,
                                                  T *__restrict__ y, int64_t rows, int64_t D,
                                                  float eps, int vec_ok) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const T *xr = x + row * D;
    T *yr = y + row * D;
    float ss = 0.0f;
    const bool vec = (sizeof(T) == 2) && vec_ok;
    if (vec) {
        for (int64_t c = lane; c < D / 8; c += 64) {
            float f[8];
            if constexpr (sizeof(T) == 2) unpack8<T>(ld16(xr + 8 * c), f);
#pragma unroll
            for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(f[i], f[i], ss);
        }
    } else {
        for (int64_t k = lane; k < D; k += 64) {
            const float v = (float)xr[k];
            ss = __builtin_fmaf(v, v, ss);
        }
    }
    ss = wave_sum(ss);
    const float inv = 1.0f / __fsqrt_rn(ss / (float)D + eps);
    if (vec) {
        for (int64_t c = lane; c < D / 8; c += 64) {
            if constexpr (sizeof(T) == 2) {
                float f[8], g[8];
                unpack8<T>(ld16(xr + 8 * c), f);
                unpack8<T>(ld16(w + 8 * c), g);
#pragma unroll
                for (int i = 0; i < 8; ++i) f[i] = g[i] * (float)cvt<T>(pin32<T>(f[i] * inv));
                st16(yr + 8 * c, pack8<T>(f));
            }
        }
    } else {
        for (int64_t k = lane; k < D; k += 64)
            yr[k] = cvt<T>((float)w[k] * (float)cvt<T>(pin32<T>((float)xr[k] * inv)));
    }
}

// Wide rows (16-bit T, D % 8 == 0, D <= 8 * 256 * RC): one 256-thread
// workgroup per row, the row held in registers between the sum of squares and
// the scaled store, so x is read once and every load is issued up front.
// Same arithmetic as rms_kernel: fma sum of squares in chunk order per
// thread, then a fixed-order reduction (xor tree in each wave, waves 0..3).
constexpr int RMS_RC = 2;  // 16-byte chunks per thread

// The normalization of one row whose 16-byte chunks c = threadIdx.x + 256 i
// (c < nc) this thread holds in xv, with the weight chunks in wv.
template <typename T>
__device__ __forceinline__ void rms_row_store(const uint4 (&xv)[RMS_RC],
                                              const uint4 (&wv)[RMS_RC], T *__restrict__ yr,
                                              int nc, int64_t D, float eps) {
    __shared__ float part[4];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < RMS_RC; ++i) {
        if (threadIdx.x + 256 * i < nc) {
            float f[8];
            unpack8<T>(xv[i], f);
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(f[e], f[e], ss);
        }
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = ((part[0] + part[1]) + part[2]) + part[3];
    const float inv = 1.0f / __fsqrt_rn(ss / (float)D + eps);
#pragma unroll
    for (int i = 0; i < RMS_RC; ++i) {
        const int c = threadIdx.x + 256 * i;
        if (c < nc) {
            float f[8], g[8];
            unpack8<T>(xv[i], f);
            unpack8<T>(wv[i], g);
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = g[e] * (float)cvt<T>(pin32<T>(f[e] * inv));
            st16(yr + 8 * c, pack8<T>(f));
        }
    }
}

template <typename T>
__global__ __launch_bounds__(256) void rms_row_kernel(const T *__restrict__ x,
                                                      const T *__restrict__ w, T *__restrict__ y,
                                                      int64_t D, float eps) {
    const int64_t row = blockIdx.x;
    const T *xr = x + row * D;
    const int nc = (int)(D / 8);
    uint4 xv[RMS_RC], wv[RMS_RC];
    // the weight is loaded with the row, not after the reduction: one memory
    // round trip per launch instead of two
#pragma unroll
    for (int i = 0; i < RMS_RC; ++i) {
        const int c = threadIdx.x + 256 * i;
        const int cc = c < nc ? c : nc - 1;  // clamped: in bounds, unused past nc
        xv[i] = ld16(xr + 8 * cc);
        wv[i] = ld16(w + 8 * cc);
    }
    rms_row_store<T>(xv, wv, y + row * D, nc, D, eps);
}

// [qmm, add, rms_norm] after a K-part launch: row m of h is
// T(resid + T(sum of the KS fp32 parts, in part order)), the [qmm, add]
// epilogue, and the normalized row is rms_row_kernel's on that h (the same
// chunks per thread, so the same sums). One workgroup per row. Every load of
// a thread (its chunks of each part, the residual and the weight) is issued
// before the first add: a loop over a run-time part count had waited for each
// part's loads in turn, one memory round trip per part and chunk.
template <typename T, int KS>
__global__ __launch_bounds__(256) void rms_parts_kernel(const float *__restrict__ part,
                                                        const T *__restrict__ resid,
                                                        const T *__restrict__ w,
                                                        T *__restrict__ h, T *__restrict__ y,
                                                        int64_t M, int64_t D, float eps) {
    const int64_t row = blockIdx.x;
    const int nc = (int)(D / 8);
    uint4 xv[RMS_RC], wv[RMS_RC], rv[RMS_RC];
    float4 pv[RMS_RC][KS][2];
#pragma unroll
    for (int i = 0; i < RMS_RC; ++i) {
        const int c = threadIdx.x + 256 * i;
        const int cc = c < nc ? c : nc - 1;  // clamped: in bounds, unused past nc
        const int64_t o = row * D + 8 * cc;
#pragma unroll
        for (int z = 0; z < KS; ++z) {
            pv[i][z][0] = *(const float4 *)(part + z * M * D + o);
            pv[i][z][1] = *(const float4 *)(part + z * M * D + o + 4);
        }
        rv[i] = ld16(resid + o);
        wv[i] = ld16(w + 8 * cc);
    }
#pragma unroll
    for (int i = 0; i < RMS_RC; ++i) {
        const int c = threadIdx.x + 256 * i;
        const float4 lo = pv[i][0][0], hi = pv[i][0][1];
        float s[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
        for (int z = 1; z < KS; ++z) {
            s[0] += pv[i][z][0].x;
            s[1] += pv[i][z][0].y;
            s[2] += pv[i][z][0].z;
            s[3] += pv[i][z][0].w;
            s[4] += pv[i][z][1].x;
            s[5] += pv[i][z][1].y;
            s[6] += pv[i][z][1].z;
            s[7] += pv[i][z][1].w;
        }
        float f[8];
        unpack8<T>(rv[i], f);
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = pin32<T>(f[e] + (float)cvt<T>(s[e]));
        xv[i] = pack8<T>(f);
        if (c < nc) st16(h + row * D + 8 * c, xv[i]);
    }
    rms_row_store<T>(xv, wv, y + row * D, nc, D, eps);
}

// rms_row_kernel's shapes: 16-bit rows of 1024..4096 values, 16-byte aligned
inline bool rms_row_ok(int64_t D, const void *x, const void *w, const void *y) {
    return D % 8 == 0 && D >= 1024 && D <= 8 * 256 * RMS_RC && aligned(x, 16) && aligned(w, 16) &&
           aligned(y, 16);
}

template <typename T>
int launch_rms(const void *x, const void *w, void *y, int64_t rows, int64_t D, float eps,
               hipStream_t st) {
    if (rows == 0) return MI_OK;
    const int vec = D % 8 == 0 && aligned(x, 16) && aligned(w, 16) && aligned(y, 16);
    if constexpr (sizeof(T) == 2) {
        if (rms_row_ok(D, x, w, y)) {
            rms_row_kernel<T><<<(unsigned)rows, 256, 0, st>>>((const T *)x, (const T *)w,
                                                              (T *)y, D, eps);
            return launch_status("rms_norm");
        }
    }
    rms_kernel<T><<<(unsigned)ceil_div(rows, 4), 256, 0, st>>>((const T *)x, (const T *)w,
                                                                (T *)y, rows, D, eps, vec);
    return launch_status("rms_norm");
}

// One row = one head vector of D values, owned by R lanes (R a power of two).
// Slot p < dims/2 is a rotated pair; slots past it copy two tail values.
// One launch serves up to three jobs (the attention prologue's q, k and v):
// each job has its own input (row stride xs), norm weight (NULL: no norm),
// head count, output [B, H, cap, D] at rows pos0.., and rope dims (0: none).
// Rows are numbered job 0 first, then 1, then 2.
struct NRJob {
    const void *x, *w;
    void *out;
    int64_t H, xs, cap, pos0;
    int dims;
};
struct NRJobs {
    NRJob j0, j1, j2;
    int64_t end0, end1, rows;  // cumulative row ends
};

// R lanes per row. VEC (16-bit T, D == 8 R, every row 16-byte aligned): each
// lane owns four rotation pairs (elements 4t..4t+3 and their partners D/2
// on), moved as 8-byte loads and stores, or eight consecutive elements of a
// row that is only normalized or copied; otherwise R = D / 2 and a lane owns
// one pair (or the general loop runs).
template <typename T, int R, bool VEC>
__global__ __launch_bounds__(256) void norm_rope_kernel(NRJobs jobs, int64_t B, int64_t L,
                                                        int64_t D, float eps, int trad,
                                                        float log2base, float scale,
                                                        int64_t offset) {
    const int t = threadIdx.x % R;
    int64_t row = (int64_t)blockIdx.x * (256 / R) + threadIdx.x / R;
    if (row >= jobs.rows) return;
    // the row's job, selected field by field (no indexed copy of the table)
    const bool a0 = row < jobs.end0, a1 = !a0 && row < jobs.end1;
    row -= a0 ? 0 : (a1 ? jobs.end0 : jobs.end1);
    const T *x = (const T *)(a0 ? jobs.j0.x : (a1 ? jobs.j1.x : jobs.j2.x));
    const T *w = (const T *)(a0 ? jobs.j0.w : (a1 ? jobs.j1.w : jobs.j2.w));
    T *out = (T *)(a0 ? jobs.j0.out : (a1 ? jobs.j1.out : jobs.j2.out));
    const int64_t H = a0 ? jobs.j0.H : (a1 ? jobs.j1.H : jobs.j2.H);
    const int64_t xs = a0 ? jobs.j0.xs : (a1 ? jobs.j1.xs : jobs.j2.xs);
    const int64_t cap = a0 ? jobs.j0.cap : (a1 ? jobs.j1.cap : jobs.j2.cap);
    const int64_t pos0 = a0 ? jobs.j0.pos0 : (a1 ? jobs.j1.pos0 : jobs.j2.pos0);
    const int dims = a0 ? jobs.j0.dims : (a1 ? jobs.j1.dims : jobs.j2.dims);
    // (32-bit: rows < 2^31; a 64-bit division per lane costs tens of VALU)
    const unsigned ur = (unsigned)row, uh = (unsigned)H, ul = (unsigned)L;
    const int64_t h = ur % uh, l = (ur / uh) % ul, b = ur / (uh * ul);
    const T *xr = x + (b * L + l) * xs + h * D;
    T *orow = out + ((b * H + h) * cap + pos0 + l) * D;
    const int half = dims / 2;
    const int slots = (int)(D / 2);
    const float position = (float)(l + offset) * scale;
    if constexpr (VEC) {
        if (!trad && dims == D) {
            // four pairs per lane: one sum of squares over the lane's eight
            // elements, a butterfly over the row's R lanes, the same
            // normalization and rotation per element as below
            const int e0 = 4 * t, hd = (int)(D / 2);
            const uint2 xa = ld8(xr + e0), xc = ld8(xr + hd + e0);
            const uint2 wa = w ? ld8(w + e0) : make_uint2(0, 0);
            const uint2 wc = w ? ld8(w + hd + e0) : make_uint2(0, 0);
            float sn[4], cs[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float inv_freq = exp2f(-(float)(2 * (e0 + e)) / (float)dims * log2base);
                sincosf(position * inv_freq, &sn[e], &cs[e]);
            }
            float a[4], c[4];
            unpack4<T>(xa, a);
            unpack4<T>(xc, c);
            if (w) {
                float ss = 0.0f;
#pragma unroll
                for (int e = 0; e < 4; ++e) ss = __builtin_fmaf(a[e], a[e], ss);
#pragma unroll
                for (int e = 0; e < 4; ++e) ss = __builtin_fmaf(c[e], c[e], ss);
#pragma unroll
                for (int o = R / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o, R);
                const float inv = 1.0f / __fsqrt_rn(ss / (float)D + eps);
                float ga[4], gc[4];
                unpack4<T>(wa, ga);
                unpack4<T>(wc, gc);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    a[e] = (float)cvt<T>(ga[e] * (float)cvt<T>(pin32<T>(a[e] * inv)));
                    c[e] = (float)cvt<T>(gc[e] * (float)cvt<T>(pin32<T>(c[e] * inv)));
                }
            }
            float r0[4], r1[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                r0[e] = pin32<T>(rope_first(a[e], c[e], cs[e], sn[e]));
                r1[e] = pin32<T>(rope_second(a[e], c[e], cs[e], sn[e]));
            }
            st8(orow + e0, pack4<T>(r0));
            st8(orow + hd + e0, pack4<T>(r1));
            return;
        }
        if (dims == 0) {  // no rotation: the normalized row, or a plain copy
            const uint4 xv = ld16(xr + 8 * t);
            if (!w) {
                st16(orow + 8 * t, xv);
                return;
            }
            const uint4 wv = ld16(w + 8 * t);
            float f[8], g[8];
            unpack8<T>(xv, f);
            unpack8<T>(wv, g);
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(f[e], f[e], ss);
#pragma unroll
            for (int o = R / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o, R);
            const float inv = 1.0f / __fsqrt_rn(ss / (float)D + eps);
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = (float)cvt<T>(g[e] * (float)cvt<T>(pin32<T>(f[e] * inv)));
            st16(orow + 8 * t, pack8<T>(f));
            return;
        }
    }
    if (!VEC && !trad && D == 2 * R && dims == D) {
        // Each lane owns elements t and t + R: its two terms of the RMS and
        // one rotation pair. One load of each, issued with the weights before
        // the angle math, which then runs under their latency; the same
        // arithmetic, in the same order, as the general loop below.
        const float a0 = (float)xr[t], c0 = (float)xr[t + R];
        const float wa = w ? (float)w[t] : 1.0f, wc = w ? (float)w[t + R] : 1.0f;
        const float inv_freq = exp2f(-(float)(2 * t) / (float)dims * log2base);
        float sn, cs;
        sincosf(position * inv_freq, &sn, &cs);
        float a = a0, c = c0;
        if (w) {
            float ss = __builtin_fmaf(a0, a0, 0.0f);
            ss = __builtin_fmaf(c0, c0, ss);
#pragma unroll
            for (int o = R / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o, R);
            const float inv = 1.0f / __fsqrt_rn(ss / (float)D + eps);
            a = (float)cvt<T>(wa * (float)cvt<T>(pin32<T>(a0 * inv)));
            c = (float)cvt<T>(wc * (float)cvt<T>(pin32<T>(c0 * inv)));
        }
        orow[t] = cvt<T>(pin32<T>(rope_first(a, c, cs, sn)));
        orow[t + R] = cvt<T>(pin32<T>(rope_second(a, c, cs, sn)));
        return;
    }
    float inv = 1.0f;
    if (w) {
        float ss = 0.0f;
        for (int k = t; k < D; k += R) {
            const float v = (float)xr[k];
            ss = __builtin_fmaf(v, v, ss);
        }
#pragma unroll
        for (int o = R / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o, R);
        inv = 1.0f / __fsqrt_rn(ss / (float)D + eps);
    }
    for (int p = t; p < slots; p += R) {
        int e0, e1;
        const bool rot = p < half;
        if (trad || !rot) {
            e0 = rot ? 2 * p : dims + 2 * (p - half);
            e1 = e0 + 1;
        } else {
            e0 = p;
            e1 = p + half;
        }
        float a = (float)xr[e0], c = (float)xr[e1];
        if (w) {
            a = (float)cvt<T>((float)w[e0] * (float)cvt<T>(pin32<T>(a * inv)));
            c = (float)cvt<T>((float)w[e1] * (float)cvt<T>(pin32<T>(c * inv)));
        }
        if (rot) {
            const float inv_freq = exp2f(-(float)(2 * p) / (float)dims * log2base);
            float sn, cs;
            sincosf(position * inv_freq, &sn, &cs);
            const float ra = pin32<T>(rope_first(a, c, cs, sn));
            const float rc = pin32<T>(rope_second(a, c, cs, sn));
            a = ra;
            c = rc;
        }
        orow[e0] = cvt<T>(a);
        orow[e1] = cvt<T>(c);
    }
}

template <typename T>
int launch_norm_rope(const NRJobs &jobs, int64_t B, int64_t L, int64_t D, float eps, int trad,
                     float log2base, float scale, int64_t offset, hipStream_t st) {
    const int64_t rows = jobs.rows;
    if (rows == 0) return MI_OK;
    if (rows >= ((int64_t)1 << 31))  // the kernel splits a row index in 32 bits
        return fail(MI_ERR_UNSUPPORTED, "norm_rope of %lld rows", (long long)rows);
    const int64_t slots = D / 2;
#define MI_NR_LAUNCH(RR, V)                                                                    \
    norm_rope_kernel<T, RR, V><<<(unsigned)ceil_div(rows, 256 / RR), 256, 0, st>>>(             \
        jobs, B, L, D, eps, trad, log2base, scale, offset)
    // 16-byte rows: every job's x, weight and output base 16-byte aligned and
    // its x row stride a multiple of 8 elements (D itself is)
    auto row16 = [&](const NRJob &j) {
        return aligned(j.x, 16) && aligned(j.w, 16) && aligned(j.out, 16) && j.xs % 8 == 0;
    };
    if constexpr (sizeof(T) == 2) {
        const bool vec = D >= 64 && D <= 512 && (D & (D - 1)) == 0 && row16(jobs.j0) &&
                         row16(jobs.j1) && row16(jobs.j2);
        if (vec) {
            if (D == 512)
                MI_NR_LAUNCH(64, true);
            else if (D == 256)
                MI_NR_LAUNCH(32, true);
            else if (D == 128)
                MI_NR_LAUNCH(16, true);
            else
                MI_NR_LAUNCH(8, true);
            return launch_status("norm_rope");
        }
    }
    if (slots >= 64)
        MI_NR_LAUNCH(64, false);
    else if (slots >= 32)
        MI_NR_LAUNCH(32, false);
    else if (slots >= 16)
        MI_NR_LAUNCH(16, false);
    else
        MI_NR_LAUNCH(8, false);
#undef MI_NR_LAUNCH
    return launch_status("norm_rope");
}

}  // namespace

int rms_launch(const void *x, const void *w, void *y, int64_t rows, int64_t D, float eps,
               int dtype, void *stream) {
    if (!valid_dtype(dtype)) return fail(MI_ERR_UNSUPPORTED, "dtype code %d", dtype);
    if (rows < 0 || D <= 0) return fail(MI_ERR_ARG, "rms_norm shape rows=%lld D=%lld",
                                        (long long)rows, (long long)D);
    if (rows && (!x || !w || !y)) return fail(MI_ERR_ARG, "null pointer");
    hipStream_t st = as_stream(stream);
    switch (dtype) {
    case MI_BF16: return launch_rms<bf16>(x, w, y, rows, D, eps, st);
    case MI_F16: return launch_rms<f16>(x, w, y, rows, D, eps, st);
    default: return launch_rms<float>(x, w, y, rows, D, eps, st);
    }
}

}  // namespace mi

using namespace mi;

extern "C" int mi_rms_norm(const void *x, const void *w, void *y, int64_t rows, int64_t D,
                           float eps, int dtype, void *stream) {
    return rms_launch(x, w, y, rows, D, eps, dtype, stream);
}

extern "C" int mi_qmm_affine_residual_rmsnorm(const void *x, const uint32_t *w,
                                              const void *scales, const void *biases,
                                              const void *resid, const void *norm_w, float eps,
                                              void *h, void *y, int64_t M, int64_t N, int64_t K,
                                              int group_size, int bits, int dtype,
                                              void *stream) {
    if (M && N && (!norm_w || !y)) return fail(MI_ERR_ARG, "null norm weight or output");
    if (int e = qmm_residual_launch(x, w, scales, biases, resid, h, M, N, K, group_size, bits,
                                    dtype, stream))
        return e;
    if (M == 0 || N == 0) return MI_OK;
    return rms_launch(h, norm_w, y, M, N, eps, dtype, stream);
}

extern "C" int mi_qmm_affine_residual_rmsnorm_ws(const void *x, const uint32_t *w,
                                                 const void *scales, const void *biases,
                                                 const void *resid, const void *norm_w, float eps,
                                                 void *h, void *y, int64_t M, int64_t N, int64_t K,
                                                 int group_size, int bits, int dtype,
                                                 void *workspace, int64_t workspace_bytes,
                                                 void *stream) {
    const int64_t need = qmm_parts_bytes(M, N, K, group_size, bits, dtype);
    if (need == 0 || !workspace || workspace_bytes < need || !aligned(workspace, 16) ||
        !rms_row_ok(N, h, norm_w, y) || !aligned(resid, 16))
        return mi_qmm_affine_residual_rmsnorm(x, w, scales, biases, resid, norm_w, eps, h, y, M,
                                              N, K, group_size, bits, dtype, stream);
    if (!norm_w || !y || !h || !resid)
        return fail(MI_ERR_ARG, "null norm weight, output or residual");
    if (int e = qmm_parts_launch(x, w, scales, biases, (float *)workspace, M, N, K, group_size,
                                 bits, dtype, stream))
        return e;
    const int ks = (int)(need / (M * N * (int64_t)sizeof(float)));
    hipStream_t st = as_stream(stream);
#define MI_RMS_PARTS(TT, KS)                                                                   \
    rms_parts_kernel<TT, KS><<<(unsigned)M, 256, 0, st>>>((const float *)workspace,              \
                                                          (const TT *)resid, (const TT *)norm_w, \
                                                          (TT *)h, (TT *)y, M, N, eps)
    if (ks == 4 && dtype == MI_BF16)
        MI_RMS_PARTS(bf16, 4);
    else if (ks == 4)
        MI_RMS_PARTS(f16, 4);
    else
        return fail(MI_ERR_UNSUPPORTED, "%d K parts", ks);
#undef MI_RMS_PARTS
    return launch_status("qmm + residual + rms_norm (sum of K parts)");
}

namespace mi {
namespace {

// Checks one job and appends it to the table (rows numbered in job order).
int add_job(NRJobs &jobs, int n, const void *x, const void *w, void *out, int64_t B, int64_t L,
            int64_t H, int64_t D, int64_t xs, int dims, int64_t cap, int64_t pos) {
    if (B < 0 || L < 0 || H <= 0 || D <= 0 || D % 2)
        return fail(MI_ERR_ARG, "norm_rope shape B=%lld L=%lld H=%lld D=%lld", (long long)B,
                    (long long)L, (long long)H, (long long)D);
    if (dims < 0 || dims > D || dims % 2)
        return fail(MI_ERR_ARG, "rope dims %d vs head dim %lld", dims, (long long)D);
    if (xs < H * D) return fail(MI_ERR_ARG, "x row stride smaller than H*D");
    if (pos < 0 || pos + L > cap)
        return fail(MI_ERR_ARG, "rows [%lld, %lld) exceed the output capacity %lld",
                    (long long)pos, (long long)(pos + L), (long long)cap);
    if (B * L && (!x || !out)) return fail(MI_ERR_ARG, "null pointer");
    const NRJob j = {x, w, out, H, xs, cap, pos, dims};
    const int64_t start = jobs.rows;
    jobs.rows += B * L * H;
    if (n == 0) {
        jobs.j0 = jobs.j1 = jobs.j2 = j;
        jobs.end0 = jobs.end1 = jobs.rows;
    } else if (n == 1) {
        jobs.j1 = jobs.j2 = j;
        jobs.end0 = start;
        jobs.end1 = jobs.rows;
    } else {
        jobs.j2 = j;
        jobs.end1 = start;
    }
    return MI_OK;
}

int run_norm_rope(const NRJobs &jobs, int64_t B, int64_t L, int64_t D, float eps, int dims,
                  int trad, float base, float scale, int64_t offset, int dtype, void *stream) {
    if (dims && !(base > 0.0f)) return fail(MI_ERR_ARG, "rope base must be positive");
    const float log2base = dims ? (float)log2((double)base) : 0.0f;
    hipStream_t st = as_stream(stream);
    switch (dtype) {
    case MI_BF16:
        return launch_norm_rope<bf16>(jobs, B, L, D, eps, trad, log2base, scale, offset, st);
    case MI_F16:
        return launch_norm_rope<f16>(jobs, B, L, D, eps, trad, log2base, scale, offset, st);
    default:
        return launch_norm_rope<float>(jobs, B, L, D, eps, trad, log2base, scale, offset, st);
    }
}

}  // namespace
}  // namespace mi

extern "C" int mi_norm_rope(const void *x, const void *w, void *out, int64_t B, int64_t L,
                            int64_t H, int64_t D, int64_t x_row_stride, float eps, int rope_dims,
                            int traditional, float base, float scale, int64_t offset,
                            int64_t out_seq_cap, int64_t out_pos, int dtype, void *stream) {
    if (!valid_dtype(dtype)) return fail(MI_ERR_UNSUPPORTED, "dtype code %d", dtype);
    NRJobs jobs = {};
    if (int e = add_job(jobs, 0, x, w, out, B, L, H, D, x_row_stride, rope_dims, out_seq_cap,
                        out_pos))
        return e;
    return run_norm_rope(jobs, B, L, D, eps, rope_dims, traditional, base, scale, offset, dtype,
                         stream);
}

extern "C" int mi_norm_rope_qkv(const void *q, const void *k, const void *v, int64_t q_row_stride,
                                int64_t k_row_stride, int64_t v_row_stride, const void *q_norm,
                                const void *k_norm, void *q_out, void *k_cache, void *v_cache,
                                int64_t B, int64_t L, int64_t Hq, int64_t Hkv, int64_t D,
                                float eps, int rope_dims, int traditional, float base,
                                float scale, int64_t offset, int64_t kv_cap, int64_t kv_pos,
                                int dtype, void *stream) {
    if (!valid_dtype(dtype)) return fail(MI_ERR_UNSUPPORTED, "dtype code %d", dtype);
    NRJobs jobs = {};
    if (int e = add_job(jobs, 0, q, q_norm, q_out, B, L, Hq, D, q_row_stride, rope_dims, L, 0))
        return e;
    if (int e = add_job(jobs, 1, k, k_norm, k_cache, B, L, Hkv, D, k_row_stride, rope_dims,
                        kv_cap, kv_pos))
        return e;
    if (int e = add_job(jobs, 2, v, nullptr, v_cache, B, L, Hkv, D, v_row_stride, 0, kv_cap,
                        kv_pos))
        return e;
    return run_norm_rope(jobs, B, L, D, eps, rope_dims, traditional, base, scale, offset, dtype,
                         stream);
}
