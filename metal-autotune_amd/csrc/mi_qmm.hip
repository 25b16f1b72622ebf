// Rows A2-A4 (+ the A5/A8/A9 region epilogues): affine quantized matmul.
//
// y[M, N] = x[M, K] @ dequant(w)^T with w uint32 [N, K*bits/32] (MLX layout),
// scales/biases T [N, K/gs]. Two kernels, mirroring the library's two regimes
// (scaffold/stitch.py:74-100, 176-293):
//
//  * qmv_kernel (small M, and the generic fallback): 16 lanes per output row,
//    4 rows per wave; each lane streams 16-byte weight chunks and accumulates
//    the per-group factored sum s*sum(x*q) + b*sum(x) in fp32
//    (lower.py:1179-1233); a 16-lane xor-shuffle tree reduces the row.
//
//  * qmm_mfma_kernel (M > 8, bf16/fp16): 32x32x16 MFMA with the weight tile
//    as the A operand (rows = output features) and x^T as B (columns =
//    tokens), so each lane ends with 4 consecutive output features of one
//    token (8-byte stores). A lane's A fragment for one MFMA is 8 consecutive
//    k of one weight row: exactly one packed word at 4 bits. Weights are loaded
//    16 bytes per lane (4 words) and the 4 words feed 4 successive MFMAs by
//    permuting k inside the 64-wide "super-step": lane half h covers
//    k0 + 32h .. k0 + 32h + 31 and MFMA step j takes the 8 values
//    k0 + 32h + 8j .. +7, for both operands. Each weight element is
//    dequantized once per kernel (T(fma(s, q, b)), the A1 form) in registers
//    -- no LDS for weights. Waves split K inside the workgroup (WK) so a
//    128-token tile still spans 256 CUs' worth of work at N = 9728; partial
//    tiles are reduced through LDS in a fixed order (deterministic).
//
// Epilogues implement the reference's region cuts: plain store; [qmm, add];
// [qmm, split(3), mul]; [qmm(w1), qmm(w3)] (two outputs, or swiglu fused).
#include "mi_common.h"

namespace mi {
namespace {

enum Epi { EPI_STORE = 0, EPI_RESID = 1, EPI_SPLIT3 = 2, EPI_DUAL = 3, EPI_SWIGLU = 4 };

constexpr int epi_parts(int e) { return e == EPI_SPLIT3 ? 3 : (e >= EPI_DUAL ? 2 : 1); }

struct QParams {
    const void *x;             // T [M, K]
    const uint32_t *w[3];      // packed weights per part
    const void *s[3];          // scales per part
    const void *b[3];          // biases per part
    int64_t noff[3];           // row offset of each part inside its weight
    const void *resid;         // T [M, Nout] (EPI_RESID)
    void *y0;                  // T [M, Nout]
    void *y1;                  // T [M, Nout] (EPI_SPLIT3, EPI_DUAL)
    int64_t M, Nout, K;
    int gs;
    int wk;                    // K-split waves (qmm_mfma_kernel)
};

template <typename T> __device__ __forceinline__ float swiglu1(float g, float u) {
    const float gt = (float)cvt<T>(g);
    const float sig = (float)cvt<T>(1.0f / (1.0f + __expf(-gt)));
    const float act = (float)cvt<T>(gt * sig);
    return act * (float)cvt<T>(u);
}

// Epilogue for one output element (m, n) of the output sub-space.
template <typename T, int EPI>
__device__ __forceinline__ void epi1(const QParams &p, int64_t m, int64_t n, const float *acc) {
    T *y0 = (T *)p.y0;
    const int64_t o = m * p.Nout + n;
    if constexpr (EPI == EPI_STORE) {
        y0[o] = cvt<T>(acc[0]);
    } else if constexpr (EPI == EPI_RESID) {
        y0[o] = cvt<T>((float)((const T *)p.resid)[o] + (float)cvt<T>(acc[0]));
    } else if constexpr (EPI == EPI_SPLIT3) {
        // split(3): parts 0, 1, 2 are B, C, x; outputs C and T(B * x)
        y0[o] = cvt<T>(acc[1]);
        ((T *)p.y1)[o] = cvt<T>((float)cvt<T>(acc[0]) * (float)cvt<T>(acc[2]));
    } else if constexpr (EPI == EPI_DUAL) {
        y0[o] = cvt<T>(acc[0]);
        ((T *)p.y1)[o] = cvt<T>(acc[1]);
    } else {
        y0[o] = cvt<T>(swiglu1<T>(acc[0], acc[1]));
    }
}

// Epilogue for 4 consecutive output features n..n+3 of token m; acc[part][e].
template <typename T, int EPI, int P>
__device__ __forceinline__ void epi4(const QParams &p, int64_t m, int64_t n,
                                     const float (&acc)[P][4]) {
    if (m >= p.M || n >= p.Nout) return;
    if (n + 4 > p.Nout || (p.Nout & 3)) {  // ragged tail: element stores
        for (int e = 0; e < 4 && n + e < p.Nout; ++e) {
            float a[P];
#pragma unroll
            for (int q = 0; q < P; ++q) a[q] = acc[q][e];
            epi1<T, EPI>(p, m, n + e, a);
        }
        return;
    }
    const int64_t o = m * p.Nout + n;
    float v[4];
    if constexpr (EPI == EPI_STORE) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[0][e];
    } else if constexpr (EPI == EPI_RESID) {
        const uint2 rr = ld8((const T *)p.resid + o);
        typedef typename Vec<T>::x4 V4;
        const V4 rv = __builtin_bit_cast(V4, rr);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (float)rv[e] + (float)cvt<T>(acc[0][e]);
    } else if constexpr (EPI == EPI_SPLIT3) {
        float bx[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = acc[1][e];
            bx[e] = (float)cvt<T>(acc[0][e]) * (float)cvt<T>(acc[2][e]);
        }
        st8((T *)p.y1 + o, pack4<T>(bx));
    } else if constexpr (EPI == EPI_DUAL) {
        float u[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = acc[0][e];
            u[e] = acc[1][e];
        }
        st8((T *)p.y1 + o, pack4<T>(u));
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = swiglu1<T>(acc[0][e], acc[1][e]);
    }
    st8((T *)p.y0 + o, pack4<T>(v));
}

// ---------------------------------------------------------------------------
// GEMV / generic path

template <typename T, int VPC>
__device__ __forceinline__ void load_x(const T *xp, float (&xf)[VPC]) {
    if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int i = 0; i < VPC; i += 4) {
            const uint4 r = ld16(xp + i);
            xf[i] = __uint_as_float(r.x);
            xf[i + 1] = __uint_as_float(r.y);
            xf[i + 2] = __uint_as_float(r.z);
            xf[i + 3] = __uint_as_float(r.w);
        }
    } else {
#pragma unroll
        for (int i = 0; i < VPC; i += 8) {
            float f[8];
            unpack8<T>(ld16(xp + i), f);
#pragma unroll
            for (int j = 0; j < 8; ++j) xf[i + j] = f[j];
        }
    }
}

template <typename T, int BITS, int MR, int EPI>
__global__ __launch_bounds__(256) void qmv_kernel(QParams p) {
    constexpr int P = epi_parts(EPI);
    constexpr int VPW = 32 / BITS;
    constexpr int VPC = 4 * VPW;
    const int lane = threadIdx.x & 63;
    const int j = lane & 15;
    const int64_t n = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 6) * 4 + (lane >> 4);
    const int64_t m0 = (int64_t)blockIdx.y * MR;
    const int64_t K = p.K, cpr = K / VPC, G = K / p.gs;
    const int mr = (int)((p.M - m0) < MR ? (p.M - m0) : MR);
    const T *x = (const T *)p.x + m0 * K;

    float acc[P][MR];
#pragma unroll
    for (int q = 0; q < P; ++q)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[q][m] = 0.0f;

    if (n < p.Nout) {
        const uint32_t *wr[P];
        const T *sr[P];
        const T *br[P];
#pragma unroll
        for (int q = 0; q < P; ++q) {
            const int64_t row = p.noff[q] + n;
            wr[q] = p.w[q] + row * (K / VPW);
            sr[q] = (const T *)p.s[q] + row * G;
            br[q] = (const T *)p.b[q] + row * G;
        }
#pragma unroll 2
        for (int64_t c = j; c < cpr; c += 16) {
            const int64_t k0 = c * VPC;
            float qf[P][VPC];
            float sc[P], bi[P];
#pragma unroll
            for (int q = 0; q < P; ++q) {
                const uint4 wv = ld16(wr[q] + c * 4);
                const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
                for (int i = 0; i < VPC; ++i)
                    qf[q][i] = (float)((words[i / VPW] >> ((i % VPW) * BITS)) &
                                       ((1u << BITS) - 1u));
                sc[q] = (float)sr[q][k0 / p.gs];
                bi[q] = (float)br[q][k0 / p.gs];
            }
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                if (m < mr) {
                    float xf[VPC];
                    load_x<T, VPC>(x + m * K + k0, xf);
                    float dx = 0.0f;
#pragma unroll
                    for (int i = 0; i < VPC; ++i) dx += xf[i];
#pragma unroll
                    for (int q = 0; q < P; ++q) {
                        float dq = 0.0f;
#pragma unroll
                        for (int i = 0; i < VPC; ++i) dq = __builtin_fmaf(xf[i], qf[q][i], dq);
                        acc[q][m] += sc[q] * dq + bi[q] * dx;
                    }
                }
            }
        }
    }
#pragma unroll
    for (int q = 0; q < P; ++q)
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            float v = acc[q][m];
            v += __shfl_xor(v, 8, 16);
            v += __shfl_xor(v, 4, 16);
            v += __shfl_xor(v, 2, 16);
            v += __shfl_xor(v, 1, 16);
            acc[q][m] = v;
        }
    if (j == 0 && n < p.Nout) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            if (m < mr) {
                float a[P];
#pragma unroll
                for (int q = 0; q < P; ++q) a[q] = acc[q][m];
                epi1<T, EPI>(p, m0 + m, n, a);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// MFMA path

template <typename T> struct Mfma;
template <> struct Mfma<bf16> {
    static __device__ __forceinline__ f32x16 mma(bf16x8 a, bf16x8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};
template <> struct Mfma<f16> {
    static __device__ __forceinline__ f32x16 mma(f16x8 a, f16x8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

// A: 32-row weight tiles per wave (one per part when P > 1); C: 32-token
// tiles per wave; WN: waves along N; WKMAX: the largest K split (p.wk <= it).
template <typename T, int BITS, int A, int C, int WN, int WKMAX, int EPI>
__global__ __launch_bounds__(64 * WN * WKMAX) void qmm_mfma_kernel(QParams p) {
    constexpr int P = epi_parts(EPI);
    static_assert(P == 1 || A == P, "multi-part epilogues use one tile per part");
    constexpr int TN = (P == 1) ? A : 1;  // 32-wide output tiles per wave
    constexpr int VPW = 32 / BITS;        // values per word
    constexpr int VPC = 4 * VPW;          // values per 16-byte chunk (per lane half)
    constexpr int S = VPC / 8;            // MFMA steps per super-step
    constexpr int SS = 2 * VPC;           // k per super-step
    typedef typename Vec<T>::x8 V8;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wn = wave % WN, kw = wave / WN;
    const int h = lane >> 5, r = lane & 31;
    const int64_t K = p.K, G = K / p.gs;
    const int64_t n_wave = (int64_t)blockIdx.x * (32 * TN * WN) + wn * 32 * TN;
    const int64_t m_blk = (int64_t)blockIdx.y * (32 * C);
    const int wk = p.wk;
    const int64_t Kw = K / wk;
    const int64_t kbeg = kw * Kw;
    const int nsteps = (int)(Kw / SS);

    const uint32_t *wrow[A];
    const T *srow[A];
    const T *brow[A];
    bool wok[A];
#pragma unroll
    for (int a = 0; a < A; ++a) {
        const int part = (P == 1) ? 0 : a;
        const int64_t nout = n_wave + ((P == 1) ? 32 * a : 0) + r;
        wok[a] = nout < p.Nout;
        const int64_t row = p.noff[part] + (wok[a] ? nout : 0);
        wrow[a] = p.w[part] + row * (K / VPW) + 4 * h;
        srow[a] = (const T *)p.s[part] + row * G;
        brow[a] = (const T *)p.b[part] + row * G;
    }
    const T *xrow[C];
    bool xok[C];
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int64_t m = m_blk + 32 * c + r;
        xok[c] = m < p.M;
        xrow[c] = (const T *)p.x + (xok[c] ? m : 0) * K + h * VPC;
    }

    f32x16 acc[A][C];
#pragma unroll
    for (int a = 0; a < A; ++a)
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[a][c][i] = 0.0f;

    // software pipeline: fragments of step t+1 load while step t computes
    uint4 wv[A], wn_[A];
    float sv[A], bv[A], sn[A], bn[A];
    uint4 xv[C][S], xn[C][S];
    auto load = [&](int64_t k0, uint4 (&wd)[A], float (&sd)[A], float (&bd)[A],
                    uint4 (&xd)[C][S]) {
#pragma unroll
        for (int a = 0; a < A; ++a) {
            wd[a] = wok[a] ? ld16(wrow[a] + k0 / VPW) : make_uint4(0, 0, 0, 0);
            const int64_t g = (k0 + h * VPC) / p.gs;
            sd[a] = wok[a] ? (float)srow[a][g] : 0.0f;
            bd[a] = wok[a] ? (float)brow[a][g] : 0.0f;
        }
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int j = 0; j < S; ++j)
                xd[c][j] = xok[c] ? ld16(xrow[c] + k0 + 8 * j) : make_uint4(0, 0, 0, 0);
    };
    if (nsteps > 0) load(kbeg, wv, sv, bv, xv);
    for (int t = 0; t < nsteps; ++t) {
        if (t + 1 < nsteps) load(kbeg + (int64_t)(t + 1) * SS, wn_, sn, bn, xn);
#pragma unroll
        for (int j = 0; j < S; ++j) {
#pragma unroll
            for (int a = 0; a < A; ++a) {
                const uint32_t words[4] = {wv[a].x, wv[a].y, wv[a].z, wv[a].w};
                const V8 af = (BITS == 4)
                                  ? dequant8<T, 4>(words[j], 0u, sv[a], bv[a])
                                  : dequant8<T, 8>(words[2 * j], words[2 * j + 1], sv[a], bv[a]);
#pragma unroll
                for (int c = 0; c < C; ++c)
                    acc[a][c] = Mfma<T>::mma(af, __builtin_bit_cast(V8, xv[c][j]), acc[a][c]);
            }
        }
        if (t + 1 < nsteps) {
#pragma unroll
            for (int a = 0; a < A; ++a) {
                wv[a] = wn_[a];
                sv[a] = sn[a];
                bv[a] = bn[a];
            }
#pragma unroll
            for (int c = 0; c < C; ++c)
#pragma unroll
                for (int j = 0; j < S; ++j) xv[c][j] = xn[c][j];
        }
    }

    if constexpr (WKMAX > 1) {
        // fixed-order reduction of the K-split partial tiles through LDS
        constexpr int REGS = A * C * 16;
        __shared__ float red[(WKMAX - 1) * WN * REGS * 64];
        if (wk > 1) {
            if (kw > 0) {
                float *dst = red + ((size_t)((kw - 1) * WN + wn) * REGS) * 64 + lane;
#pragma unroll
                for (int a = 0; a < A; ++a)
#pragma unroll
                    for (int c = 0; c < C; ++c)
#pragma unroll
                        for (int i = 0; i < 16; ++i) dst[((a * C + c) * 16 + i) * 64] = acc[a][c][i];
            }
            __syncthreads();
            if (kw > 0) return;
            for (int src = 1; src < wk; ++src) {
                const float *s = red + ((size_t)((src - 1) * WN + wn) * REGS) * 64 + lane;
#pragma unroll
                for (int a = 0; a < A; ++a)
#pragma unroll
                    for (int c = 0; c < C; ++c)
#pragma unroll
                        for (int i = 0; i < 16; ++i) acc[a][c][i] += s[((a * C + c) * 16 + i) * 64];
            }
        }
    }

    // D[row][col] of a 32x32 tile: col = lane % 32 (token), row = 8*(i/4) +
    // 4*(lane/32) + i%4 (feature): 4 consecutive features per (i/4) block.
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int64_t m = m_blk + 32 * c + r;
#pragma unroll
        for (int blk = 0; blk < 4; ++blk) {
            if constexpr (P == 1) {
#pragma unroll
                for (int a = 0; a < A; ++a) {
                    float v[1][4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[0][e] = acc[a][c][4 * blk + e];
                    epi4<T, EPI, 1>(p, m, n_wave + 32 * a + 8 * blk + 4 * h, v);
                }
            } else {
                float v[P][4];
#pragma unroll
                for (int q = 0; q < P; ++q)
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[q][e] = acc[q][c][4 * blk + e];
                epi4<T, EPI, P>(p, m, n_wave + 8 * blk + 4 * h, v);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// dispatch

constexpr int QMV_MR = 8;     // rows per GEMV block (and the GEMV/MFMA switch)

template <typename T, int BITS, int EPI>
int launch_qmv(const QParams &p, hipStream_t st) {
    const dim3 grid((unsigned)ceil_div(p.Nout, 16), (unsigned)ceil_div(p.M, QMV_MR));
    if (p.M == 1)
        qmv_kernel<T, BITS, 1, EPI><<<grid, 256, 0, st>>>(p);
    else if (p.M <= 2)
        qmv_kernel<T, BITS, 2, EPI><<<grid, 256, 0, st>>>(p);
    else if (p.M <= 4)
        qmv_kernel<T, BITS, 4, EPI><<<grid, 256, 0, st>>>(p);
    else
        qmv_kernel<T, BITS, QMV_MR, EPI><<<grid, 256, 0, st>>>(p);
    return launch_status("quantized matmul (qmv)");
}

template <typename T, int BITS, int A, int C, int WN, int WKMAX, int EPI>
int launch_mfma_cfg(QParams p, int wk, hipStream_t st) {
    constexpr int P = epi_parts(EPI);
    constexpr int TN = (P == 1) ? A : 1;
    p.wk = wk;
    const dim3 grid((unsigned)ceil_div(p.Nout, 32 * TN * WN), (unsigned)ceil_div(p.M, 32 * C));
    qmm_mfma_kernel<T, BITS, A, C, WN, WKMAX, EPI><<<grid, 64 * WN * wk, 0, st>>>(p);
    return launch_status("quantized matmul (mfma)");
}

template <typename T, int BITS, int EPI>
int launch_mfma(const QParams &p, hipStream_t st) {
    constexpr int P = epi_parts(EPI);
    constexpr int A = (P == 1) ? 2 : P;
    constexpr int SS = 2 * 4 * (32 / BITS);
    const int64_t ks = p.K / SS;  // super-steps
    const int wk = (ks % 4 == 0) ? 4 : (ks % 2 == 0 ? 2 : 1);
    if (p.M > 256) return launch_mfma_cfg<T, BITS, A, 4, 4, 1, EPI>(p, 1, st);
    if (p.M > 64) return launch_mfma_cfg<T, BITS, A, 4, 1, 4, EPI>(p, wk, st);
    if (p.M > 32) return launch_mfma_cfg<T, BITS, A, 2, 1, 4, EPI>(p, wk, st);
    return launch_mfma_cfg<T, BITS, A, 1, 1, 4, EPI>(p, wk, st);
}

template <typename T, int EPI>
int launch_typed(const QParams &p, int bits, hipStream_t st) {
    const int SS = 2 * 4 * (32 / bits);
    const bool mfma = (sizeof(T) == 2) && p.M > QMV_MR && (p.K % SS == 0);
    if constexpr (sizeof(T) == 2) {
        if (mfma)
            return bits == 4 ? launch_mfma<T, 4, EPI>(p, st) : launch_mfma<T, 8, EPI>(p, st);
    }
    return bits == 4 ? launch_qmv<T, 4, EPI>(p, st) : launch_qmv<T, 8, EPI>(p, st);
}

template <int EPI>
int run(const QParams &p, int bits, int dtype, void *stream) {
    if (p.M == 0 || p.Nout == 0) return MI_OK;
    hipStream_t st = as_stream(stream);
    switch (dtype) {
    case MI_BF16: return launch_typed<bf16, EPI>(p, bits, st);
    case MI_F16: return launch_typed<f16, EPI>(p, bits, st);
    default: return launch_typed<float, EPI>(p, bits, st);
    }
}

QParams base_params(const void *x, const uint32_t *w, const void *s, const void *b, void *y,
                    int64_t M, int64_t Nout, int64_t K, int gs) {
    QParams p = {};
    p.x = x;
    for (int i = 0; i < 3; ++i) {
        p.w[i] = w;
        p.s[i] = s;
        p.b[i] = b;
        p.noff[i] = 0;
    }
    p.y0 = y;
    p.M = M;
    p.Nout = Nout;
    p.K = K;
    p.gs = gs;
    p.wk = 1;
    return p;
}

int check_common(const void *x, const void *w, const void *s, const void *b, const void *y,
                 int64_t M, int64_t N, int64_t K, int gs, int bits, int dtype) {
    if (int e = check_quant(N, K, gs, bits, dtype)) return e;
    if (M < 0) return fail(MI_ERR_ARG, "negative M");
    if (M && N && (!x || !w || !s || !b || !y)) return fail(MI_ERR_ARG, "null pointer");
    if (!aligned(x, 16) || !aligned(w, 16) || !aligned(y, 8))
        return fail(MI_ERR_ARG, "x and w must be 16-byte aligned, outputs 8-byte aligned");
    return MI_OK;
}

}  // namespace

int qmm_residual_launch(const void *x, const uint32_t *w, const void *s, const void *b,
                        const void *resid, void *y, int64_t M, int64_t N, int64_t K, int gs,
                        int bits, int dtype, void *stream) {
    if (int e = check_common(x, w, s, b, y, M, N, K, gs, bits, dtype)) return e;
    if (M && N && !resid) return fail(MI_ERR_ARG, "null residual");
    if (!aligned(resid, 8)) return fail(MI_ERR_ARG, "residual must be 8-byte aligned");
    QParams p = base_params(x, w, s, b, y, M, N, K, gs);
    p.resid = resid;
    return run<EPI_RESID>(p, bits, dtype, stream);
}

}  // namespace mi

using namespace mi;

extern "C" int mi_qmm_affine(const void *x, const uint32_t *w, const void *scales,
                             const void *biases, void *y, int64_t M, int64_t N, int64_t K,
                             int group_size, int bits, int dtype, void *stream) {
    if (int e = check_common(x, w, scales, biases, y, M, N, K, group_size, bits, dtype)) return e;
    return run<EPI_STORE>(base_params(x, w, scales, biases, y, M, N, K, group_size), bits, dtype,
                          stream);
}

extern "C" int mi_qmm_affine_residual(const void *x, const uint32_t *w, const void *scales,
                                      const void *biases, const void *resid, void *y, int64_t M,
                                      int64_t N, int64_t K, int group_size, int bits, int dtype,
                                      void *stream) {
    return qmm_residual_launch(x, w, scales, biases, resid, y, M, N, K, group_size, bits, dtype,
                               stream);
}

extern "C" int mi_qmm_affine_split_gate(const void *x, const uint32_t *w, const void *scales,
                                        const void *biases, void *c_out, void *bx_out, int64_t M,
                                        int64_t N3, int64_t K, int group_size, int bits,
                                        int dtype, void *stream) {
    if (int e = check_common(x, w, scales, biases, c_out, M, N3, K, group_size, bits, dtype))
        return e;
    if (N3 % 3) return fail(MI_ERR_ARG, "split(3) needs N divisible by 3, got %lld", (long long)N3);
    if (M && N3 && !bx_out) return fail(MI_ERR_ARG, "null output");
    if (!aligned(bx_out, 8)) return fail(MI_ERR_ARG, "outputs must be 8-byte aligned");
    const int64_t D = N3 / 3;
    QParams p = base_params(x, w, scales, biases, c_out, M, D, K, group_size);
    p.y1 = bx_out;
    p.noff[0] = 0;
    p.noff[1] = D;
    p.noff[2] = 2 * D;
    return run<EPI_SPLIT3>(p, bits, dtype, stream);
}

extern "C" int mi_qmm_affine_dual(const void *x, const uint32_t *w1, const void *s1,
                                  const void *b1, const uint32_t *w2, const void *s2,
                                  const void *b2, void *y1, void *y2, int64_t M, int64_t N,
                                  int64_t K, int group_size, int bits, int act, int dtype,
                                  void *stream) {
    if (int e = check_common(x, w1, s1, b1, y1, M, N, K, group_size, bits, dtype)) return e;
    if (M && N && (!w2 || !s2 || !b2)) return fail(MI_ERR_ARG, "null second weight");
    if (act != MI_ACT_NONE && act != MI_ACT_SWIGLU)
        return fail(MI_ERR_UNSUPPORTED, "dual qmm activation %d", act);
    if (act == MI_ACT_NONE && M && N && !y2) return fail(MI_ERR_ARG, "null second output");
    if (!aligned(w2, 16) || !aligned(y2, 8)) return fail(MI_ERR_ARG, "misaligned second operand");
    QParams p = base_params(x, w1, s1, b1, y1, M, N, K, group_size);
    p.w[1] = w2;
    p.s[1] = s2;
    p.b[1] = b2;
    p.y1 = y2;
    if (act == MI_ACT_SWIGLU) return run<EPI_SWIGLU>(p, bits, dtype, stream);
    return run<EPI_DUAL>(p, bits, dtype, stream);
}
