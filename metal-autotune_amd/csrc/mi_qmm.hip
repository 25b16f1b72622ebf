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
// [qmm, split(3), mul]; [qmm(w1), qmm(w3)] (two outputs, or swiglu fused);
// and three projections sharing x in one launch (EPI_GROUP3: the weights and
// outputs are concatenated along N and each workgroup's tile lies in one part);
// the same three projections with the attention prologue fused (EPI_HEADNR:
// each workgroup owns one 128-value head of q, k or v for 32 tokens and applies
// the q/k RMSNorm, RoPE and the transposed cache write to its sums).
#include <math.h>

#include "mi_common.h"

namespace mi {
namespace {

enum Epi { EPI_STORE = 0, EPI_RESID = 1, EPI_SPLIT3 = 2, EPI_DUAL = 3, EPI_SWIGLU = 4,
           EPI_GROUP3 = 5, EPI_HEADNR = 6 };

// weight rows each output element combines (EPI_GROUP3 selects one weight per tile)
constexpr int epi_parts(int e) {
    return e == EPI_SPLIT3 ? 3 : ((e == EPI_DUAL || e == EPI_SWIGLU) ? 2 : 1);
}

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
    int64_t pn[3];             // EPI_GROUP3: N of each part (Nout = their sum)
    void *py[3];               // EPI_GROUP3: output of each part, T [M, pn[i]]
    int gs;
    int gs_log2;               // log2(gs): group sizes are powers of two
    int wk;                    // K-split waves (qmm_mfma_kernel)
    int sbp;                   // qmm_mfma_kernel: groups per row of a wave's scale/bias table
    int n4;                    // qmm_mfma_mixed_kernel: feature tiles taken as 128-token tiles
    int sbninst;               // qmm_mfma_kernel: DMA instructions per scale/bias table array
    unsigned sbmagic;          // ceil(2^20 / (sbp / 2)): v / (sbp / 2) as (v * sbmagic) >> 20
    int ks;                    // K parts (kpart_count): each is split over the wk waves
    int kslice;                // k values a scale/bias table covers (a wave chunk, or all of K)
    int kint;                  // interleaved K split (kint_of): wave w takes stages w, w + wk, ...
    float *part;               // non-null: write K part blockIdx.z's sums, fp32 [ks, M, Nout]
    // EPI_HEADNR (the parts are q, k, v; py[] = q_out [B, Hq, L, D], k_cache,
    // v_cache [B, Hkv, cap, D]; D = 128)
    const void *nw[2];         // q_norm, k_norm: T [D]
    int64_t L;                 // tokens per sequence (M = B L)
    int64_t cap, pos0;         // cache rows per head; first row written
    int64_t offset;            // RoPE position of a sequence's token 0
    float eps, log2base, rscale;
};

// K parts of the MFMA path: a function of (M, K) alone, so every entry point
// and epilogue (and the tile shape) gives an output element the same sums in
// the same order. Narrow-N projections at prefill sizes (o_proj, down_proj:
// N = 2560, K = 4096 / 9728, M = 128) otherwise fill 160-320 workgroups,
// each wave streaming 16-38 stages one after another. With a workspace the
// parts run as workgroups of their own (grid z) and a second kernel adds them
// in part order; without one a workgroup runs its parts in turn (qmm_mfma_tile)
// and the sums are the same. Four parts for both shapes (measured in the
// Qwen3 prefill step: o_proj with 4 parts of 64-feature tiles beats 2 parts of
// 32-feature tiles; down_proj with 8 parts loses 6 us a layer).
constexpr int KPARTS = 4;
inline int kpart_count(int64_t M, int64_t K) {
    return (M <= 8 || M > 128 || K < 4096) ? 1 : KPARTS;
}

template <typename T> __device__ __forceinline__ float swiglu1(float g, float u) {
    const float gt = (float)cvt<T>(g);
    const float sig = (float)cvt<T>(1.0f / (1.0f + __expf(-gt)));
    const float act = (float)cvt<T>(gt * sig);
    return act * (float)cvt<T>(u);
}

// The arrays one workgroup reads and writes, held as scalar fields with
// select accessors: the kernels never modify the QParams argument (a modified
// copy whose arrays are indexed in loops ends up in scratch memory).
struct Bound {
    const uint32_t *w0, *w1, *w2;
    const void *s0, *s1, *s2;
    const void *b0, *b1, *b2;
    int64_t o0, o1, o2;  // row offset of each part inside its weight
    void *y0;            // this workgroup's output
    int64_t Nout;        // its width
    int gp;              // EPI_GROUP3 / EPI_HEADNR: the part it lies in
    __device__ const uint32_t *w(int i) const { return i == 0 ? w0 : (i == 1 ? w1 : w2); }
    __device__ const void *s(int i) const { return i == 0 ? s0 : (i == 1 ? s1 : s2); }
    __device__ const void *b(int i) const { return i == 0 ? b0 : (i == 1 ? b1 : b2); }
    __device__ int64_t noff(int i) const { return i == 0 ? o0 : (i == 1 ? o1 : o2); }
};

// Binds a workgroup whose first output feature is nb. EPI_GROUP3: the three
// weights and outputs are concatenated along N and the host guarantees every
// part's N is a multiple of each tile width, so the whole tile lies in one
// part: bind that part as part 0 and make nb relative to it.
template <int EPI>
__device__ __forceinline__ Bound bind(const QParams &p, int64_t &nb) {
    Bound q = {p.w[0], p.w[1], p.w[2], p.s[0], p.s[1], p.s[2], p.b[0], p.b[1], p.b[2],
               p.noff[0], p.noff[1], p.noff[2], p.y0, p.Nout, 0};
    if constexpr (EPI == EPI_GROUP3 || EPI == EPI_HEADNR) {
        const int64_t e0 = p.pn[0], e1 = p.pn[0] + p.pn[1];
        const bool p0 = nb < e0, p1 = !p0 && nb < e1;
        nb -= p0 ? 0 : (p1 ? e0 : e1);
        q.w0 = p0 ? p.w[0] : (p1 ? p.w[1] : p.w[2]);
        q.s0 = p0 ? p.s[0] : (p1 ? p.s[1] : p.s[2]);
        q.b0 = p0 ? p.b[0] : (p1 ? p.b[1] : p.b[2]);
        q.y0 = p0 ? p.py[0] : (p1 ? p.py[1] : p.py[2]);
        q.Nout = p0 ? p.pn[0] : (p1 ? p.pn[1] : p.pn[2]);
        q.gp = p0 ? 0 : (p1 ? 1 : 2);
    }
    return q;
}

// Epilogue for one output element (m, n) of the output sub-space.
template <typename T, int EPI>
__device__ __forceinline__ void epi1(const QParams &p, const Bound &bd, int64_t m, int64_t n,
                                     const float *acc) {
    T *y0 = (T *)bd.y0;
    const int64_t o = m * bd.Nout + n;
    if constexpr (EPI == EPI_STORE || EPI == EPI_GROUP3 || EPI == EPI_HEADNR) {
        y0[o] = cvt<T>(acc[0]);
    } else if constexpr (EPI == EPI_RESID) {
        y0[o] = cvt<T>(pin32<T>((float)((const T *)p.resid)[o] + (float)cvt<T>(acc[0])));
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

// Whether epi4 takes its vector path at (m, n): in range, four whole features.
__device__ __forceinline__ bool epi4_vec(const QParams &p, const Bound &bd, int64_t m, int64_t n) {
    return m < p.M && n + 4 <= bd.Nout && !(bd.Nout & 3);
}

// EPI_RESID: the residual's four values at (m, n) for epi4's vector path,
// loaded ahead so a wave's loads are all in flight before its first store
// (each epi4 loading its own had waited for every load in turn); zeros where
// the vector path does not run (the element path loads its own).
template <typename T>
__device__ __forceinline__ uint2 resid4(const QParams &p, const Bound &bd, int64_t m, int64_t n) {
    return epi4_vec(p, bd, m, n) ? ld8((const T *)p.resid + m * bd.Nout + n) : make_uint2(0u, 0u);
}

// Epilogue for 4 consecutive output features n..n+3 of token m; acc[part][e].
// rpre: EPI_RESID's residual from resid4 (null: loaded here).
template <typename T, int EPI, int P>
__device__ __forceinline__ void epi4(const QParams &p, const Bound &bd, int64_t m, int64_t n,
                                     const float (&acc)[P][4], const uint2 *rpre = nullptr) {
    if (m >= p.M || n >= bd.Nout) return;
    if (n + 4 > bd.Nout || (bd.Nout & 3)) {  // ragged tail: element stores
        for (int e = 0; e < 4 && n + e < bd.Nout; ++e) {
            float a[P];
#pragma unroll
            for (int q = 0; q < P; ++q) a[q] = acc[q][e];
            epi1<T, EPI>(p, bd, m, n + e, a);
        }
        return;
    }
    const int64_t o = m * bd.Nout + n;
    float v[4];
    if constexpr (EPI == EPI_STORE || EPI == EPI_GROUP3 || EPI == EPI_HEADNR) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[0][e];
    } else if constexpr (EPI == EPI_RESID) {
        const uint2 rr = rpre ? *rpre : ld8((const T *)p.resid + o);
        typedef typename Vec<T>::x4 V4;
        const V4 rv = __builtin_bit_cast(V4, rr);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = pin32<T>((float)rv[e] + (float)cvt<T>(acc[0][e]));
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
    st8((T *)bd.y0 + o, pack4<T>(v));
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
    int64_t nb = (int64_t)blockIdx.x * 16;
    const Bound bd = bind<EPI>(p, nb);
    const int64_t n = nb + (threadIdx.x >> 6) * 4 + (lane >> 4);
    const int64_t m0 = (int64_t)blockIdx.y * MR;
    const int64_t K = p.K, cpr = K / VPC, G = K >> p.gs_log2;
    const int mr = (int)((p.M - m0) < MR ? (p.M - m0) : MR);
    const T *x = (const T *)p.x + m0 * K;

    float acc[P][MR];
#pragma unroll
    for (int q = 0; q < P; ++q)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[q][m] = 0.0f;

    // out-of-range rows/tokens read clamped, valid addresses (no branch around
    // loads); their sums are never stored
    const int64_t nrow = n < bd.Nout ? n : bd.Nout - 1;
    const uint32_t *wr[P];
    const T *sr[P];
    const T *br[P];
#pragma unroll
    for (int q = 0; q < P; ++q) {
        const int64_t row = bd.noff(q) + nrow;
        wr[q] = bd.w(q) + row * (K / VPW);
        sr[q] = (const T *)bd.s(q) + row * G;
        br[q] = (const T *)bd.b(q) + row * G;
    }
#pragma unroll 2
    for (int64_t c = j; c < cpr; c += 16) {
        const int64_t k0 = c * VPC;
        float qf[P][VPC];
        float sc[P], bi[P];
#pragma unroll
        for (int q = 0; q < P; ++q) {
            const uint4 wv = ld16_nt(wr[q] + c * 4);
            const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
            for (int i = 0; i < VPC; ++i)
                qf[q][i] =
                    (float)((words[i / VPW] >> ((i % VPW) * BITS)) & ((1u << BITS) - 1u));
            sc[q] = (float)sr[q][k0 >> p.gs_log2];
            bi[q] = (float)br[q][k0 >> p.gs_log2];
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            float xf[VPC];
            load_x<T, VPC>(x + (m < mr ? m : mr - 1) * K + k0, xf);
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
#pragma unroll
    for (int q = 0; q < P; ++q)
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            acc[q][m] = row16_sum(acc[q][m]);  // the row's 16 lanes
        }
    if (j == 0 && n < bd.Nout) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            if (m < mr) {
                float a[P];
#pragma unroll
                for (int q = 0; q < P; ++q) a[q] = acc[q][m];
                epi1<T, EPI>(p, bd, m0 + m, n, a);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Decode GEMV (M <= 4, 4-bit, bf16/fp16): the nibbles never go through a
// float conversion. (w >> 4j) & 0x000F000F | MAGIC packs nibbles j and j+4 of a
// word as the two 16-bit floats MAG + q exactly (bf16: 0x4300 = 128, ulp 1 up
// to 256; fp16: 0x6400 = 1024, ulp 1), so one v_and_or makes a pair and
// v_dot2_f32_{bf16,f16} multiplies it with the x pair (x[k], x[k+4]):
//   sum_k x_k (MAG + q_k) = D  ->  s*sum(x q) + b*sum(x) = s*D + (b - MAG*s)*sum(x).
// x is staged once per workgroup in LDS already permuted into those pairs,
// with per-32-value chunk sums. Weight chunks are loaded 8 per lane before use.

template <typename T> struct Magic;
template <> struct Magic<bf16> {
    static constexpr uint32_t pair = 0x43004300u;
    static constexpr float value = 128.0f;
    static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
        typedef __bf16 v2 __attribute__((ext_vector_type(2)));
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b),
                                               c, false);
    }
};
template <> struct Magic<f16> {
    static constexpr uint32_t pair = 0x64006400u;
    static constexpr float value = 1024.0f;
    static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
        typedef _Float16 v2 __attribute__((ext_vector_type(2)));
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c,
                                      false);
    }
};

// ((w >> 4j) & 0x000F000F) | Mg::pair -- the magic pair of nibbles j and
// j + 4 of w -- in fewer instructions: the even and odd nibbles as bytes
// (lo, hi) once per word, then one byte permute per pair that interleaves two
// of those bytes with the magic exponent byte. Same bits.
template <typename T>
__device__ __forceinline__ uint32_t magic_pair(uint32_t w, int j) {
    constexpr uint32_t e = (Magic<T>::pair >> 8) & 0xFFu;  // the exponent byte (0x43 / 0x64)
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    // v_perm_b32 bytes: 0..3 from the second operand, 4..7 from the first
    const uint32_t sel = (j & 2) ? 0x04030401u : 0x04020400u;
    return __builtin_amdgcn_perm(e * 0x01010101u, (j & 1) ? hi : lo, sel);
}

constexpr int QV_BATCH = 8;  // 16-byte weight chunks in flight per lane

inline int64_t qmv_dot2_lds_bytes(int mr, int64_t K) { return mr * K * 2 + mr * (K / 32) * 4; }

// A workgroup of blockDim.x / 64 waves owns 64 / LPR output rows per wave (LPR
// lanes a row, below): 4 waves, or for single-output epilogues without PF up
// to 16 (WIDE), sized by the host so the grid spreads the rows evenly over the
// CUs. Wider workgroups are not used for the others: batches of two or three
// weight rows take more than the 128 registers a lane may hold in a 16-wave
// workgroup, and under PF the staging barriers wait for the x loads of every
// wave, which queue behind the weight stream (one 10-wave workgroup per CU at
// N = 9728 waited 2.3 us for x against 1.5 us with 4 waves: 6.1 against 5.6
// us a launch).
// PF (4 waves at 16 lanes a row; also wide workgroups of a row a wave): the x
// loads, then the first weight batch, are issued before x is staged, so the
// weight stream runs under the staging and its two barriers (x first: vmcnt
// retires in issue order, so waiting for x then leaves the weights in
// flight). Each thread holds at most two x chunks (K / 8 <= 2 blockDim.x). It
// costs the batch registers through the staging, which pays when the grid
// fits the chip in one round and not at N = 151936.
constexpr bool qmv_dot2_wide_ok(int epi) { return epi_parts(epi) == 1 && epi != EPI_GROUP3; }

// LPR: lanes per output row, 16 (4 rows a wave) or 64 (a row a wave, for long
// K: a K = 9728 row is 19 chunks a lane at 16 lanes, loaded in three batches
// one after another, and about 5 at 64, one batch).
template <typename T, int MR, int EPI, bool PF = false, bool WIDE = false, int LPR = 16>
__global__ __launch_bounds__(WIDE ? 1024 : 256) void qmv_dot2_kernel(QParams p) {
    static_assert(!WIDE || qmv_dot2_wide_ok(EPI), "wide workgroups: single output");
    static_assert(LPR == 16 || (LPR == 64 && qmv_dot2_wide_ok(EPI)), "a row a wave: single output");
    static_assert(!PF || MR == 1, "PF: one token");
    static_assert(!PF || !WIDE || LPR == 64, "PF in wide workgroups: a row a wave");
    constexpr int RPW = 64 / LPR;  // rows a wave
    constexpr int P = epi_parts(EPI);
    typedef Magic<T> Mg;
    extern __shared__ uint4 xs_pairs[];  // [MR][K/8] pair blocks, then [MR][K/32] sums
    const int64_t K = p.K, words = K / 8, cpr = K / 32, G = K >> p.gs_log2;
    float *xsum = (float *)(xs_pairs + MR * words);
    const int lane = threadIdx.x & 63, j = lane & (LPR - 1);
    const int bs = WIDE ? (int)blockDim.x : 256;  // threads
    int64_t nb = (int64_t)blockIdx.x * ((bs >> 6) * RPW);
    const Bound bd = bind<EPI>(p, nb);
    const int64_t n = nb + (threadIdx.x >> 6) * RPW + lane / LPR;
    const int64_t nrow = n < bd.Nout ? n : bd.Nout - 1;
    const int64_t m0 = (int64_t)blockIdx.y * MR;
    const int mr = (int)((p.M - m0) < MR ? (p.M - m0) : MR);

    const uint32_t *wr[P];
    const T *sr[P];
    const T *br[P];
#pragma unroll
    for (int q = 0; q < P; ++q) {
        const int64_t row = bd.noff(q) + nrow;
        wr[q] = bd.w(q) + row * (K / 8);
        sr[q] = (const T *)bd.s(q) + row * G;
        br[q] = (const T *)bd.b(q) + row * G;
    }

    uint4 wv[P][QV_BATCH];
    T sv[P][QV_BATCH], bv[P][QV_BATCH];
    auto load_batch = [&](int64_t base) {
#pragma unroll
        for (int i = 0; i < QV_BATCH; ++i) {
            const int64_t c = base + LPR * i;
            const int64_t cc = c < cpr ? c : cpr - 1;
            const int64_t g = (cc * 32) >> p.gs_log2;
#pragma unroll
            for (int q = 0; q < P; ++q) {
                wv[q][i] = ld16_nt(wr[q] + 4 * cc);
                sv[q][i] = sr[q][g];
                bv[q][i] = br[q][g];
            }
        }
    };

    // stage x rows as pairs (e[i], e[i+4]) of each 8-value block
    const T *x = (const T *)p.x + m0 * K;
    auto pairs = [](const uint4 d) {
        return make_uint4(__builtin_amdgcn_perm(d.z, d.x, 0x05040100u),
                          __builtin_amdgcn_perm(d.z, d.x, 0x07060302u),
                          __builtin_amdgcn_perm(d.w, d.y, 0x05040100u),
                          __builtin_amdgcn_perm(d.w, d.y, 0x07060302u));
    };
    const int nw = (int)words;  // 32-bit index math: MR * K < 2^31
    if constexpr (PF) {
        // Every thread issues both loads (a clamped, valid chunk when past the
        // end) so the issue order, and with it the waits, is the same in all
        // waves: x, then the weights (K / 8 <= 2 bs)
        uint4 d[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            int idx = (int)threadIdx.x + bs * t;
            idx = idx < MR * nw ? idx : MR * nw - 1;
            const int m = MR == 1 ? 0 : idx / nw, w = idx - m * nw;
            d[t] = ld16(x + (int64_t)(m < mr ? m : mr - 1) * K + 8 * w);
        }
        __builtin_amdgcn_sched_barrier(0);  // keep the x loads ahead of the weights'
        load_batch(j);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int64_t idx = threadIdx.x + bs * t;
            if (idx < MR * words) xs_pairs[idx] = pairs(d[t]);
        }
    } else {
        for (int idx = threadIdx.x; idx < MR * nw; idx += bs) {
            const int m = MR == 1 ? 0 : idx / nw, w = idx - m * nw;
            xs_pairs[idx] = pairs(ld16(x + (int64_t)(m < mr ? m : mr - 1) * K + 8 * w));
        }
    }
    __syncthreads();
    const int ncpr = (int)cpr;
    for (int idx = threadIdx.x; idx < MR * ncpr; idx += bs) {
        const int m = MR == 1 ? 0 : idx / ncpr, c = idx - m * ncpr;
        float s = 0.0f;
#pragma unroll
        for (int wi = 0; wi < 4; ++wi) {
            const uint4 v = xs_pairs[m * words + 4 * c + wi];
            float f[8];
            unpack8<T>(v, f);
#pragma unroll
            for (int i = 0; i < 8; ++i) s += f[i];
        }
        xsum[idx] = s;
    }
    __syncthreads();

    float acc[P][MR];
#pragma unroll
    for (int q = 0; q < P; ++q)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[q][m] = 0.0f;

    for (int64_t base = j; base < cpr; base += LPR * QV_BATCH) {
        // (Without PF the compiler sinks each chunk's loads to its use behind
        // the `c >= cpr` exit, so a lane fetches its chunks one after another;
        // at 58 registers eight waves per SIMD keep the loads in flight.)
        if (!PF || base != j) load_batch(base);
#pragma unroll
        for (int i = 0; i < QV_BATCH; ++i) {
            const int64_t c = base + LPR * i;
            if (c >= cpr) break;
#pragma unroll
            for (int q = 0; q < P; ++q) {
                const uint32_t wd[4] = {wv[q][i].x, wv[q][i].y, wv[q][i].z, wv[q][i].w};
                uint32_t qp[4][4];
#pragma unroll
                for (int wi = 0; wi < 4; ++wi)
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj)
                        qp[wi][jj] = magic_pair<T>(wd[wi], jj);
                const float s = (float)sv[q][i];
                const float bb = __builtin_fmaf(-Mg::value, s, (float)bv[q][i]);
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    float d = 0.0f;
#pragma unroll
                    for (int wi = 0; wi < 4; ++wi) {
                        const uint4 xp = xs_pairs[m * words + 4 * c + wi];
                        d = Mg::dot2(qp[wi][0], xp.x, d);
                        d = Mg::dot2(qp[wi][1], xp.y, d);
                        d = Mg::dot2(qp[wi][2], xp.z, d);
                        d = Mg::dot2(qp[wi][3], xp.w, d);
                    }
                    acc[q][m] += s * d + bb * xsum[m * cpr + c];
                }
            }
        }
    }
#pragma unroll
    for (int q = 0; q < P; ++q)
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            acc[q][m] = row16_sum(acc[q][m]);  // the row's 16 lanes
            if constexpr (LPR == 64) {  // then the wave's four 16-lane sums
                const int v = __builtin_bit_cast(int, acc[q][m]);
                const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(v, 0));
                const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(v, 16));
                const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(v, 32));
                const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(v, 48));
                acc[q][m] = (r0 + r1) + (r2 + r3);
            }
        }
    if (j == 0 && n < bd.Nout) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            if (m < mr) {
                float a[P];
#pragma unroll
                for (int q = 0; q < P; ++q) a[q] = acc[q][m];
                epi1<T, EPI>(p, bd, m0 + m, n, a);
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
// tiles per wave; WK: waves per workgroup, each owning a 1/wk slice of K.
//
// Everything a stage needs reaches a wave through LDS by direct-to-LDS DMA
// (buffer_load ... lds), into the wave's one stage slot:
//  * the x tile of the stage, 8 token rows x 128 bytes per instruction, so
//    every x cache line is fetched once (loading x fragments straight into
//    registers makes each lane read a different token row, and with four
//    waves the per-step working set overflows the 32 KB L1). The 16-byte
//    chunks of a row are XOR-swizzled by (row >> 1) & 7 so a 16-lane
//    ds_read_b128 group covers 16 distinct bank groups;
//  * each lane's 16-byte weight chunk, per part and super-step (lane l's
//    chunk lands at l * 16, where the same lane reads it back).
// The scales and biases of a wave's rows over its whole K slice are copied
// once, before the loop, into a per-wave table in dynamic LDS (sbt_layout):
// per-stage 2-byte loads touch one cache line per row for two bytes each,
// and measured on MI355X those gathers cost more load-pipeline time than the
// weights themselves.
// With no load result held in registers across stages, the explicit vmcnt
// at the top of a stage is the only wait the loop needs, and the addresses
// are a per-lane 32-bit offset plus a scalar stage offset (no VALU address
// arithmetic in the loop).
constexpr int XK = 64;  // k values per x stage (128 bytes of a token row)
constexpr int LDS_PER_CU = 160 * 1024;

template <typename T, int BITS, int A, int C, int WK>
struct MfmaShape {
    static constexpr int VPW = 32 / BITS;  // values per word
    static constexpr int VPC = 4 * VPW;    // values per 16-byte weight chunk (per lane half)
    static constexpr int S = VPC / 8;      // MFMA steps per super-step
    static constexpr int SS = 2 * VPC;     // k per super-step
    static constexpr int SPS = XK / SS;    // super-steps per x stage
    static constexpr int ROWS = 32 * C;    // token rows per stage
    static constexpr int KG = WK;          // K-groups (one wave each)
    // Several weight tiles per wave (A > 1): their chunks are prefetched one
    // stage ahead into registers instead of the slot, which keeps the slots
    // small enough for two workgroups per CU.
    static constexpr bool WREG = A > 1;
    static constexpr int XST = ROWS * 128;                           // x tile bytes per stage
    static constexpr int WAVE = WREG ? 0 : A * SPS * 1024;           // a wave's weight chunks
    static constexpr int STAGE = XST + WAVE;                         // one wave's slot
    static constexpr int XBYTES = KG * STAGE;                        // the workgroup's slots
    // K-split reduction: the partial tiles of K-groups 1..KG-1 pass through
    // the slots' LDS, RSLOTS at a time
    static constexpr int PB = A * C * 16 * 64 * 4;                   // one K-group's partials
    static constexpr int RSLOTS = KG <= 1 ? 1 : (XBYTES / PB >= KG - 1 ? KG - 1
                                                 : (XBYTES / PB > 0 ? XBYTES / PB : 1));
    static constexpr int RBYTES = RSLOTS * PB;
    static constexpr int LDS = XBYTES > RBYTES ? XBYTES : RBYTES;
    // DMA instructions a lane issues per stage: its x rows, and weights
    static constexpr int XOPS = ROWS / 8;
    static constexpr int OPS = XOPS + (WREG ? 0 : A * SPS);
    // vmcnt once the prologue (the first stage's DMAs, plus its register
    // weights) is issued: only the scale/bias table before it has landed
    static constexpr int TABLE_VMCNT = OPS + (WREG ? A * SPS : 0);
    // the stage loop is unrolled twice so the two register weight sets are
    // named statically
    static constexpr int UNROLL = 2;
    static_assert(TABLE_VMCNT < 64, "vmcnt is a 6-bit count");
    static_assert(LDS <= LDS_PER_CU, "stage slots exceed the LDS of a CU");
};

// Scale/bias table of one wave: for each of its A weight tiles, the scales
// then the biases of its 32 rows, pitch groups (2-byte values) per row,
// starting at the even group at or below the wave's first group. The pitch
// covers the wave's K slice plus the alignment group and is 2 mod 4, so the
// 32 rows' reads of one column hit 32 distinct banks. Each array is copied
// with 4-byte DMAs (two groups per lane, which needs an even number of
// groups per weight row), padded to whole 64-lane instructions.
struct SbtLayout {
    int pitch;        // groups per row
    int ninst;        // DMA instructions per array
    int array_bytes;  // ninst * 256
};
__host__ __device__ inline SbtLayout sbt_layout(int64_t kslice, int gs) {
    int need = (int)(kslice / gs) + 2;
    need += ((2 - need) % 4 + 4) % 4;
    const int ninst = (32 * need / 2 + 63) / 64;
    return {need, ninst, ninst * 256};
}

// A raw buffer resource over [base, base + bytes): 32-bit offsets, and reads
// past the end return zero instead of touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, uint32_t bytes) {
    // dword 3: 32-bit data format (gfx9 raw buffer access)
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                             0x00020000);
}

// One stage slot per wave. Measured on MI355X at the Qwen3 prefill shapes
// (M = 128), it beats rings of two to eight slots: the small footprint lets
// three workgroups share a CU (three waves per SIMD, which overlap one wave's
// dequant VALU with the others' MFMAs and loads), where two slots allowed two
// workgroups and three slots one. Dual 38.0 -> 32.9 us, q/k/v 15.0 -> 13.8,
// o_proj 12.1 -> 11.5, bit for bit the same results. (A balanced grid of one
// workgroup per CU gains nothing from deeper rings either: 25.9 us with one
// slot, 27.7 us with two or three, dual at N = 8192.)

// s_waitcnt with vmcnt = N and no wait on the other counters (gfx9 encoding:
// vmcnt[3:0] at bits 3:0 and vmcnt[5:4] at bits 15:14, expcnt 7, lgkmcnt 15).
template <int N> __device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit count");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// s_waitcnt lgkmcnt(0) with no wait on vmcnt (63) or expcnt (7)
__device__ __forceinline__ void wait_lgkmcnt0() {
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));
}

// Waves per SIMD the register allocation must allow: the single slot exists
// so three workgroups of four waves share a CU (at most 168 registers a
// lane), which tiles of up to four 32x32 accumulators fit without spilling;
// larger tiles, and 128-token tiles (whose slot alone leaves room for two
// workgroups), ask for two (256 registers).
template <int A, int C> constexpr int mfma_waves_per_eu() {
    return A * C <= 4 && C <= 2 ? 3 : 2;
}

// EPI_HEADNR epilogue. The workgroup's tile is head n_head / 128 of part
// bd.gp (0 q, 1 k, 2 v) for tokens m_blk .. m_blk + 31, computed by eight
// waves: wave (f, q) -- feature half f, K chunk q -- takes the 32-feature
// tiles at 32 f and 64 + 32 f, so after the K-split reduction it holds
// features 32 f + 64 a + 8 q + 4 h + e (a < 2, e < 4) of token m_blk + r in
// acc[a][e]. The arithmetic is norm_rope_kernel's 16-lane form on the
// T-rounded sums, which a separate launch would read back: there lane t owns
// features 4t .. 4t+3 and their RoPE partners 64 + 4t .., sums their squares
// in one fma chain (its four, then the partners) and adds the 16 lanes' sums
// in an xor butterfly (8, 4, 2, 1). Here a lane is that kernel's lane
// t = 8 f + 2 q + h with its partners in the same registers: the chain runs in
// the lane, and the butterfly pairs the token's sixteen chain sums the same
// way after an exchange through xch (16 x 32 floats of LDS). A two-operand add
// commutes exactly, so the sum, and every output, equals the separate
// launch's bit for bit. sn and cs are the sine and cosine of the rotation of
// pair (g + e, g + e + 64), g = 32 f + 8 q + 4 h, from the separate launch's
// expressions (computed in the tile's prologue).
template <typename T>
__device__ __forceinline__ void head_norm_rope(const QParams &p, const Bound &bd,
                                               const float (&acc)[2][4], const float (&sn)[4],
                                               const float (&cs)[4], int f, int q, int h, int r,
                                               int64_t m_blk, int64_t n_head, float *xch) {
    constexpr int D = 128;
    const int64_t m = m_blk + r;
    const bool live = m < p.M;
    const int64_t mm = live ? m : p.M - 1;  // (tokens past M store nothing)
    const int64_t l = mm % p.L, b = mm / p.L;
    const int part = bd.gp;  // workgroup-uniform
    const int64_t H = bd.Nout / D, hd = n_head / D;
    const int64_t cap = part == 0 ? p.L : p.cap, pos0 = part == 0 ? 0 : p.pos0;
    T *orow = (T *)bd.y0 + ((b * H + hd) * cap + pos0 + l) * D;
    const int g0 = 32 * f + 8 * q + 4 * h;  // the lane's first feature; its partners g0 + 64
    float v[2][4];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[a][e] = (float)cvt<T>(acc[a][e]);
    if (part == 2) {  // v: the cache rows as the GEMM rounds them
        if (live) {
#pragma unroll
            for (int a = 0; a < 2; ++a) st8(orow + 64 * a + g0, pack4<T>(v[a]));
        }
        return;
    }
    float ss = 0.0f;  // the separate launch's lane t = 8 f + 2 q + h
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int e = 0; e < 4; ++e) ss = __builtin_fmaf(v[a][e], v[a][e], ss);
    xch[(8 * f + 2 * q + h) * 32 + r] = ss;
    __syncthreads();
    float x[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) x[t] = xch[t * 32 + r];
    // level 8 pairs t with t ^ 8, level 4 with t ^ 4, level 2 with t ^ 2,
    // level 1 with t ^ 1
    float x1[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) x1[t] = x[t] + x[t + 8];
    const float sum = ((x1[0] + x1[4]) + (x1[2] + x1[6])) + ((x1[1] + x1[5]) + (x1[3] + x1[7]));
    const float inv = 1.0f / __fsqrt_rn(sum / (float)D + p.eps);
    const T *w = (const T *)p.nw[part];
    float gw[2][4];
#pragma unroll
    for (int a = 0; a < 2; ++a) unpack4<T>(ld8(w + 64 * a + g0), gw[a]);
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int e = 0; e < 4; ++e)
            v[a][e] = (float)cvt<T>(gw[a][e] * (float)cvt<T>(pin32<T>(v[a][e] * inv)));
    float r0[4], r1[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        r0[e] = pin32<T>(rope_first(v[0][e], v[1][e], cs[e], sn[e]));
        r1[e] = pin32<T>(rope_second(v[0][e], v[1][e], cs[e], sn[e]));
    }
    if (live) {
        st8(orow + g0, pack4<T>(r0));
        st8(orow + 64 + g0, pack4<T>(r1));
    }
}

// The same for 64-value heads (LFM2): four waves of two 32-feature tiles by
// 128 tokens (C = 4), wave q holding features 32 a + 8 q + 4 h + e of tokens
// m_blk + 32 c + r in acc[a][c][e]. norm_rope_kernel's form for D = 64 has
// 8 lanes a row, lane t owning features 4t .. 4t+3 and partners 32 + 4t ..:
// here lane t = 2q + h with a = 0 and its partners a = 1, and the butterfly
// (4, 2, 1) pairs the token's eight chain sums, exchanged through xch
// (8 x 128 floats of LDS). The angles are computed here: at the sizes this
// form serves, other workgroups' loops cover the epilogue.
template <typename T, int C>
__device__ __forceinline__ void head_norm_rope64(const QParams &p, const Bound &bd,
                                                 const f32x16 (&acc)[2][C], int q, int h, int r,
                                                 int64_t m_blk, int64_t n_head, float *xch) {
    constexpr int D = 64;
    const int part = bd.gp;  // workgroup-uniform
    const int64_t H = bd.Nout / D, hd = n_head / D;
    const int64_t cap = part == 0 ? p.L : p.cap, pos0 = part == 0 ? 0 : p.pos0;
    const int g0 = 8 * q + 4 * h;  // the lane's first feature; its partners g0 + 32
    float v[C][2][4];
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int e = 0; e < 4; ++e) v[c][a][e] = (float)cvt<T>(acc[a][c][e]);
    auto row_of = [&](int c) -> T * {
        const int64_t m = m_blk + 32 * c + r;
        const int64_t mm = m < p.M ? m : p.M - 1;
        return (T *)bd.y0 + ((mm / p.L * H + hd) * cap + pos0 + mm % p.L) * D;
    };
    if (part == 2) {  // v: the cache rows as the GEMM rounds them
#pragma unroll
        for (int c = 0; c < C; ++c) {
            if (m_blk + 32 * c + r < p.M) {
                T *orow = row_of(c);
#pragma unroll
                for (int a = 0; a < 2; ++a) st8(orow + 32 * a + g0, pack4<T>(v[c][a]));
            }
        }
        return;
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
        float ss = 0.0f;  // the separate launch's lane t = 2q + h
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int e = 0; e < 4; ++e) ss = __builtin_fmaf(v[c][a][e], v[c][a][e], ss);
        xch[(2 * q + h) * (32 * C) + 32 * c + r] = ss;
    }
    __syncthreads();
    const T *w = (const T *)p.nw[part];
    float gw[2][4];
#pragma unroll
    for (int a = 0; a < 2; ++a) unpack4<T>(ld8(w + 32 * a + g0), gw[a]);
    float inv_freq[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
        inv_freq[e] = exp2f(-(float)(2 * (g0 + e)) / (float)D * p.log2base);
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int64_t m = m_blk + 32 * c + r;
        float x[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) x[t] = xch[t * (32 * C) + 32 * c + r];
        // level 4 pairs t with t ^ 4, level 2 with t ^ 2, level 1 with t ^ 1
        const float sum = ((x[0] + x[4]) + (x[2] + x[6])) + ((x[1] + x[5]) + (x[3] + x[7]));
        const float inv = 1.0f / __fsqrt_rn(sum / (float)D + p.eps);
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                v[c][a][e] = (float)cvt<T>(gw[a][e] * (float)cvt<T>(pin32<T>(v[c][a][e] * inv)));
        const int64_t mm = m < p.M ? m : p.M - 1;
        const float position = (float)(mm % p.L + p.offset) * p.rscale;
        float r0[4], r1[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float sn, cs;
            sincosf(position * inv_freq[e], &sn, &cs);
            r0[e] = pin32<T>(rope_first(v[c][0][e], v[c][1][e], cs, sn));
            r1[e] = pin32<T>(rope_second(v[c][0][e], v[c][1][e], cs, sn));
        }
        if (m < p.M) {
            T *orow = row_of(c);
            st8(orow + g0, pack4<T>(r0));
            st8(orow + 32 + g0, pack4<T>(r1));
        }
    }
}

// One workgroup's tile: tokens [m_blk, m_blk + 32 * C) of the output features
// starting at n_blk (32 * TN of them, per part). lds is the workgroup's static
// LDS, at least MfmaShape::LDS bytes; the scale/bias tables live in the
// dynamic LDS, followed (p.ks > 1 without p.part) by the running sums over
// the K parts, mfma_sum_bytes.
//
// K is cut into p.ks * wk chunks of whole 64-value stages, chunk c covering
// stages [c T / chunks, (c + 1) T / chunks) of the T; K part z is chunks
// z wk .. z wk + wk - 1, wave kw taking chunk z wk + kw. A part's sum is
// ((c0 + c1) + c2) + c3 over its waves' chunks (the LDS reduction), and the
// output sums the parts in order, (part 0 + part 1) + .... With p.part the
// workgroup runs the one part kz and stores its sum; otherwise it runs every
// part in turn. KM selects the case at compile time (KM_ONE: ks == 1, the
// loop and its running sums compile away).
enum KMode { KM_ONE = 0, KM_LOOP = 1, KM_PART = 2 };

template <typename T, int BITS, int A, int C, int WK, int EPI, int KM = KM_ONE, int FH = 1,
          bool KI = false>
__device__ __forceinline__ void qmm_mfma_tile(const QParams &p, char *lds, int64_t n_blk,
                                              int64_t m_blk, int kz = 0) {
    // The body uses gfx950 buffer resources, which the host target cannot
    // type; the host pass needs only the kernels' launch stubs.
#if defined(__HIP_DEVICE_COMPILE__)
    typedef MfmaShape<T, BITS, A, C, WK> Sh;
    constexpr int P = epi_parts(EPI);
    static_assert(P == 1 || A == P, "multi-part epilogues use one tile per part");
    constexpr int TN = (P == 1) ? A : 1;  // 32-wide output tiles per wave
    constexpr int VPW = Sh::VPW, VPC = Sh::VPC, S = Sh::S, SS = Sh::SS, SPS = Sh::SPS;
    typedef typename Vec<T>::x8 V8;

    const int lane = threadIdx.x & 63;
    // the wave index is uniform per wave: in a scalar register, the x stage
    // base addresses and the DMA's LDS destinations (M0) need no VALU work.
    // Wave kw owns chunk kw of each K part. FH = 2 (EPI_HEADNR): eight waves,
    // wave wv taking chunk kw = wv % 4 of the 32-feature tiles at 32 fh and
    // 64 + 32 fh, fh = wv / 4 (the feature halves reduce separately).
    static_assert(FH == 1 || (FH == 2 && EPI == EPI_HEADNR && A == 2 && C == 1 && KM == KM_ONE),
                  "feature halves: the whole-head q/k/v tile only");
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kw = FH == 2 ? (wv & 3) : wv, fh = FH == 2 ? (wv >> 2) : 0;
    constexpr int TS = FH == 2 ? 64 : 32;  // row step between a wave's tiles
    const int h = lane >> 5, r = lane & 31;
    const int64_t K = p.K, G = K >> p.gs_log2;
    int64_t n_wave = n_blk;
    const Bound bd = bind<EPI>(p, n_wave);
    n_wave += 32 * fh;
    const int wk = p.wk;
    // chunks = ks * wk is a power of two (ks in {1, 4}, wk in {1, 2, 4}): chunk
    // boundaries are a shift, not a division
    const int chunks = (KM == KM_ONE ? 1 : p.ks) * wk, nstages = (int)(K / XK);
    const int cshift = __builtin_ctz((unsigned)chunks);
    const int nparts = KM == KM_LOOP ? p.ks : 1;  // K parts this workgroup runs
    char *xbuf = lds + wv * Sh::STAGE;
    const int wslot = Sh::XST;  // this wave's weights within its slot

    // Rows past N (or tokens past M) read a clamped, valid row instead of
    // branching around the load: their accumulators only feed outputs the
    // epilogue never stores. All offsets are bytes within one array, under
    // 2^32 (the host checks the sizes).
    const int gshift = p.gs_log2;
    __amdgpu_buffer_rsrc_t wr[A], sr[A], br[A];
    uint32_t woff[A];
    auto tile_row = [&](int a, int rr) -> int64_t {  // weight-array row of tile row rr
        const int part = (P == 1) ? 0 : a;
        const int64_t nout = n_wave + ((P == 1) ? TS * a : 0) + rr;
        return bd.noff(part) + (nout < bd.Nout ? nout : bd.Nout - 1);
    };
#pragma unroll
    for (int a = 0; a < A; ++a) {
        const int part = (P == 1) ? 0 : a;
        const int64_t rows = bd.noff(part) + bd.Nout;  // rows of this part's arrays
        wr[a] = buffer_rsrc(bd.w(part), (uint32_t)(rows * K * BITS / 8));
        sr[a] = buffer_rsrc(bd.s(part), (uint32_t)(rows * G * 2));
        br[a] = buffer_rsrc(bd.b(part), (uint32_t)(rows * G * 2));
        woff[a] = (uint32_t)(tile_row(a, r) * (K * BITS / 8) + 16 * h);
    }
    const int pitch = p.sbp;
    const SbtLayout tl = {pitch, p.sbninst, p.sbninst * 256};  // sbt_layout(p.kslice, p.gs)
    extern __shared__ __attribute__((aligned(16))) char lds_dyn[];
    // one scale/bias table per wave, or one for the workgroup (KI)
    static_assert(!KI || (KM == KM_ONE && FH == 1), "interleaved K split: one K part, four waves");
    const char *sbt = lds_dyn + (KI ? 0 : wv) * (A * 2 * tl.array_bytes);
    float *psum = (float *)(lds_dyn + (KI ? 1 : FH * wk) * (A * 2 * tl.array_bytes));  // sums over K parts
    typedef __attribute__((address_space(3))) void *lds_ptr;
    // x DMA: instruction i writes stage rows 8i..8i+7; lane l fills row
    // 8i + l/8 at swizzled position l%8, i.e. it loads chunk (l%8) ^ swz(row).
    // Tokens past M point past
    // the end of x's buffer resource: the load returns zeros without a memory
    // access, and every lane still issues the same instructions (the end
    // offset plus a stage offset stays below 2^32 since M * K * size < 2^31).
    const uint32_t xbytes = (uint32_t)(p.M * K * (int64_t)sizeof(T));
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(p.x, xbytes);
    // XREMAT: the 8-bit tiles with eight accumulators leave no registers for
    // the XOPS offsets (held across the loop they spilled, and every reload
    // before a DMA waited for all the DMAs in flight). Those tiles rebuild
    // offset j per stage as xrow[j % 2] + j * 8 rows: row 8j + l/8 of lane l
    // has swizzle ((4j + l/16) & 7), which depends on j only through j % 2.
    // A token past M then lies at or past xbytes by its own offset (row * K *
    // size >= M * K * size), which is the zero-returning case above; should
    // that offset wrap past 2^32 it lands inside x's buffer instead, a valid
    // read whose rows the epilogue never stores.
    constexpr bool XREMAT = BITS == 8 && A * C >= 8;
    uint32_t xoff[XREMAT ? 1 : Sh::XOPS], xrow[2];
#pragma unroll
    for (int j = 0; j < (XREMAT ? 2 : Sh::XOPS); ++j) {
        const int row = 8 * j + (lane >> 3);
        const int chunk = (lane & 7) ^ ((row >> 1) & 7);
        const uint32_t o = (uint32_t)(((m_blk + row) * K + 8 * chunk) * (int64_t)sizeof(T));
        if constexpr (XREMAT)
            xrow[j] = o;
        else
            xoff[j] = m_blk + row < p.M ? o : xbytes;
    }
    const uint32_t xrows8 = (uint32_t)(8 * K * (int64_t)sizeof(T));  // 8 token rows in bytes
    f32x16 acc[A][C];
    // EPI_HEADNR: the RoPE angles of the lane's four rotation pairs (see
    // head_norm_rope), computed while the first stage's loads are in flight
    float hsn[4], hcs[4];
    auto head_angles = [&]() {
        if constexpr (EPI == EPI_HEADNR && FH == 2) {
            const int64_t m = m_blk + r < p.M ? m_blk + r : p.M - 1;
            const float position = (float)(m % p.L + p.offset) * p.rscale;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int f = 32 * fh + 8 * kw + 4 * h + e;
                const float inv_freq = exp2f(-(float)(2 * f) / 128.0f * p.log2base);
                sincosf(position * inv_freq, &hsn[e], &hcs[e]);
                // kept here, under the loads' latency, not sunk to the epilogue
                asm volatile("" : "+v"(hsn[e]), "+v"(hcs[e]));
            }
        }
    };
    for (int kp = 0; kp < nparts; ++kp) {  // workgroup-uniform
        // The wave's stages: kbeg + st * kstep for st < nst. Contiguous
        // chunks: chunk cix of the ks * wk chunks of K. Interleaved (KI, one
        // K part, WK waves): stages kw, kw + WK, ...; a wave past the last
        // stage (K < WK * XK) runs none, and its prologue loads read the last
        // stage.
        const int cix = (KM == KM_PART ? kz : kp) * wk + kw;
        const int sbeg = (cix * nstages) >> cshift;
        const int kbeg = KI ? (kw < nstages ? kw : nstages - 1) * XK : sbeg * XK;
        const int nst = KI ? (kw < nstages ? (nstages - kw + WK - 1) / WK : 0)
                           : (((cix + 1) * nstages) >> cshift) - sbeg;
        constexpr int kstep = KI ? WK * XK : XK;
        // Scale/bias table (layout in sbt_layout): dword v of an array holds
        // groups gbase + 2j, +1 of tile row v / (pitch / 2), j = v % (pitch / 2).
        // Issued before the ring prologue, so the first stage's wait covers it.
        // KI: one table from group 0, its DMA instructions dealt to the waves
        // in turn (a barrier after the wait below).
        const int gbase = KI ? 0 : (kbeg >> gshift) & ~1;
        for (int i = KI ? kw : 0; i < tl.ninst; i += KI ? WK : 1) {
            int v = 64 * i + lane;
            v = v < 16 * pitch ? v : 16 * pitch - 1;
            const int rr = (int)(((unsigned)v * p.sbmagic) >> 20), j = v - rr * (pitch >> 1);
#pragma unroll
            for (int a = 0; a < A; ++a) {
                const uint32_t off = (uint32_t)((tile_row(a, rr) * G + gbase + 2 * j) * 2);
                char *dst = (char *)sbt + (2 * a) * tl.array_bytes + i * 256;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(sr[a], (lds_ptr)dst, 4, off, 0, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(br[a], (lds_ptr)(dst + tl.array_bytes), 4, off,
                                                         0, 0, 0);
            }
        }
        // group of value k0 + h * VPC for a super-step start k0 (a multiple of
        // 2 * VPC): k0 / gs, plus h when a group is no wider than a half-chunk;
        // as a byte offset into the table, relative to gbase
        const int hg = (p.gs <= VPC) ? h * (VPC >> gshift) : 0;
        const int sbrow = (r * pitch + hg - gbase) * 2;
        auto issue = [&](int st, char *slot) {
            const int k0 = kbeg + st * kstep;
            const uint32_t xs = (uint32_t)k0 * sizeof(T);
            if constexpr (XREMAT) {
                // opaque per stage, so the offsets are not hoisted out of the loop
                uint32_t r0 = xrow[0], r1 = xrow[1];
                launder(r0);
                launder(r1);
#pragma unroll
                for (int j = 0; j < Sh::XOPS; ++j)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(
                        xr, (lds_ptr)(slot + j * 1024), 16, ((j & 1) ? r1 : r0) + (uint32_t)(j >> 1) * 2u * xrows8,
                        xs, 0, 0);
            } else {
#pragma unroll
                for (int j = 0; j < Sh::XOPS; ++j)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_ptr)(slot + j * 1024), 16, xoff[j],
                                                             xs, 0, 0);
            }
            if constexpr (Sh::WREG) return;
#pragma unroll
            for (int u = 0; u < SPS; ++u) {
                const int ku = k0 + u * SS;
                const uint32_t ws = (uint32_t)(ku / VPW) * 4;
#pragma unroll
                for (int a = 0; a < A; ++a) {
                    char *wdst = slot + wslot + (a * SPS + u) * 1024;
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(wr[a], (lds_ptr)wdst, 16, woff[a], ws, 0, 0);
                }
            }
        };
        // WREG: the weight chunks of a stage into registers
        uint4 wreg[2][A][SPS];
        const char *wlane[A];
#pragma unroll
        for (int a = 0; a < A; ++a) {
            const int part = (P == 1) ? 0 : a;
            wlane[a] = (const char *)bd.w(part) + woff[a];
        }
        auto load_w = [&](int st, uint4 (&wd)[A][SPS]) {
#pragma unroll
            for (int u = 0; u < SPS; ++u) {
                const int ku = kbeg + st * kstep + u * SS;
                const uint32_t ws = (uint32_t)(ku / VPW) * 4;
#pragma unroll
                for (int a = 0; a < A; ++a) {
                    wd[a][u] = ld16(wlane[a] + ws);
                }
            }
        };

#pragma unroll
        for (int a = 0; a < A; ++a)
#pragma unroll
            for (int c = 0; c < C; ++c)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[a][c][i] = 0.0f;

        // Pipeline: stage st reads the wave's slot into registers, waits for those
        // reads, then refills the slot with stage st + 1 (every stage but the
        // last) and computes while those DMAs fly, so at the top of a stage
        // nothing else is in flight: vmcnt(0). (Refilling past the last stage
        // too, with a re-read of it, kept the issue pattern uniform but moved
        // 10 % more x through a CU's L1, whose outstanding requests bound the
        // x feed.) The stage loop is unrolled twice so the two register weight
        // sets are named statically.
        //
        // The slot and the scale/bias table are passed as separate __restrict__
        // arguments of the inlined main loop: the resulting alias scopes let the
        // compiler's wait-count pass see that a stage's table reads cannot touch
        // the slot the DMAs in flight are filling, so it adds no vmcnt(0) of its
        // own before them. The table's DMAs precede the prologue's, so the wait at
        // the top of stage 0 retires them.
        const int swz = (r >> 1) & 7;
        const int tab = tl.array_bytes;
        auto mainloop = [&](char *__restrict__ slot, const char *__restrict__ tb)
                            __attribute__((always_inline)) {
        const int last = nst > 0 ? nst - 1 : 0;
        // Scales and biases of a stage are read from the table one stage ahead,
        // so a stage's first dequant waits only for its weight chunk, not for the
        // x fragments read before it (LDS reads complete in order).
        uint32_t sq[A][SPS], bq[A][SPS];
        auto load_sb = [&](int st) {
#pragma unroll
            for (int a = 0; a < A; ++a)
#pragma unroll
                for (int u = 0; u < SPS; ++u) {
                    const char *sb = tb + 2 * a * tab + sbrow + ((kbeg + st * kstep + u * SS) >> gshift) * 2;
                    sq[a][u] = *(const uint16_t *)sb;
                    bq[a][u] = *(const uint16_t *)(sb + tab);
                }
        };
        issue(0, slot);
        if constexpr (Sh::WREG) load_w(0, wreg[0]);
        head_angles();
        // the table's DMAs were issued before the prologue's
        wait_vmcnt<Sh::TABLE_VMCNT>();
        if constexpr (KI) __syncthreads();  // every wave's share of the table has landed
        load_sb(0);
        for (int st0 = 0; st0 < nst; st0 += Sh::UNROLL) {
#pragma unroll
            for (int j = 0; j < Sh::UNROLL; ++j) {
                const int st = st0 + j;
                if (st >= nst) break;  // workgroup-uniform
                wait_vmcnt<0>();
                const char *cur = slot;
                // the weight chunk first: the first dequant needs it, while the
                // MFMAs that consume the x fragments come after that dequant
                uint4 wq[A][SPS];
#pragma unroll
                for (int a = 0; a < A; ++a)
#pragma unroll
                    for (int u = 0; u < SPS; ++u) {
                        if constexpr (Sh::WREG)
                            wq[a][u] = wreg[j % 2][a][u];
                        else
                            wq[a][u] = *(const uint4 *)(cur + wslot + (a * SPS + u) * 1024 + lane * 16);
                    }
                __builtin_amdgcn_sched_barrier(0);
                uint4 xf[C][SPS][S];
#pragma unroll
                for (int c = 0; c < C; ++c)
#pragma unroll
                    for (int u = 0; u < SPS; ++u)
#pragma unroll
                        for (int s = 0; s < S; ++s) {
                            const int chunk = (u * SS + h * VPC + 8 * s) >> 3;
                            xf[c][u][s] =
                                *(const uint4 *)(cur + (32 * c + r) * 128 + ((chunk ^ swz) << 4));
                        }
                // Group g = (u * S + s) * A + a is one 32-row x 16-k MFMA operand
                // and its C MFMAs. Group 0 is dequantized here, under the latency
                // of the x reads, and every later group in slices between the
                // MFMAs of the group before it (below), at both widths.
                typedef Dequant8<T, BITS> Dq;
                auto dq_init = [&](Dq &d, int g) {
                    const int u = g / (S * A), s = (g / A) % S, a = g % A;
                    const uint32_t words[4] = {wq[a][u].x, wq[a][u].y, wq[a][u].z, wq[a][u].w};
                    d.init(BITS == 4 ? words[s] : words[2 * s], BITS == 4 ? 0u : words[2 * s + 1],
                           (float)__builtin_bit_cast(T, (uint16_t)sq[a][u]),
                           (float)__builtin_bit_cast(T, (uint16_t)bq[a][u]));
                };
                uint32_t opa[4];  // the next MFMA operand: four packed pairs
                {
                    Dq d;
                    dq_init(d, 0);
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        opa[k] = d.pair(k);
                        launder(opa[k]);  // computed here, not sunk to its MFMA
                    }
                }
                // the slot's reads have returned before its refill is issued;
                // the last stage refills nothing (workgroup-uniform), so the
                // loop moves each stage's x and weights exactly once
                __builtin_amdgcn_sched_barrier(0);
                wait_lgkmcnt0();
                if (st < last) {
                    issue(st + 1, slot);
                    if constexpr (Sh::WREG) {  // one stage ahead, into the other set
                        load_w(st + 1, wreg[(j + 1) % 2]);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                // Software pipeline: each MFMA of group g is followed by a slice
                // of group g + 1's dequant (pair k after MFMA k * C / 4), so one
                // wave issues its VALU while its MFMAs run. The laundered pairs
                // and the fences keep instruction selection and the scheduler
                // from clustering the MFMAs again (they did, four at a time,
                // leaving the dequant exposed). Each accumulator still receives
                // its MFMAs in K order: the results do not change.
                constexpr int NG = SPS * S * A;
#pragma unroll
                for (int g = 0; g < NG; ++g) {
                    const int u = g / (S * A), s = (g / A) % S, a = g % A;
                    Dq d;
                    const V8 af = __builtin_bit_cast(V8, (uint4){opa[0], opa[1], opa[2], opa[3]});
#pragma unroll
                    for (int c = 0; c < C; ++c) {
                        acc[a][c] = Mfma<T>::mma(af, __builtin_bit_cast(V8, xf[c][u][s]), acc[a][c]);
                        if (g + 1 < NG) {
                            if (c == 0) {
                                dq_init(d, g + 1);
                                d.launder();
                            }
#pragma unroll
                            for (int k = 0; k < 4; ++k)
                                if ((k * C) / 4 == c) {
                                    opa[k] = d.pair(k);
                                    launder(opa[k]);
                                }
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
                load_sb(st < last ? st + 1 : last);
            }
        }
        };
        mainloop(xbuf, sbt);
        // every load has landed before the LDS is reused for the reduction or
        // released with the workgroup
        wait_vmcnt<0>();

        if constexpr (KM != KM_LOOP) {
            static_assert(Sh::KG == 4, "one-part tiles split K over four waves");
            {  // (the host launches these with wk = 4)
                // The four partial tiles reduced by all four waves. Quarter q of
                // a tile is acc[.][.][4q .. 4q+3] (features 8q + 4h .. +3 of each
                // 32x32 tile); every wave leaves the quarters it does not own in
                // LDS as 16-byte words, QPR quarters per round (as many as the
                // slots hold), and wave q adds the four copies of quarter q, its
                // own from its registers, ((p0 + p1) + p2) + p3 -- the sums of a
                // one-wave reduction -- into the registers of its own quarter 0
                // (handed over in the first round), then runs the epilogue for
                // quarter q. Each wave thus moves three quarters of its partials
                // through LDS, reads three quarters of a tile and runs a quarter
                // of the epilogue.
                constexpr int AC = A * C;
                constexpr int QPR = 4 * 4 * AC * 1024 <= Sh::LDS   ? 4
                                    : 4 * 2 * AC * 1024 <= Sh::LDS ? 2
                                                                   : 1;
                static_assert(4 * QPR * AC * 1024 <= Sh::LDS, "reduction exceeds the slots");
                // [wave][quarter in round][a * C + c][lane]; FH = 2: one region
                // per feature half (the kernel's LDS holds FH times Sh::LDS)
                float4 *red = (float4 *)(lds + fh * Sh::LDS);
                __syncthreads();  // every wave is done with its slot
#pragma unroll
                for (int q0 = 0; q0 < 4; q0 += QPR) {
                    if (q0 > 0) __syncthreads();  // the previous round's readers are done
#pragma unroll
                    for (int k = 0; k < QPR; ++k) {
                        if (kw == q0 + k) continue;  // (wave-uniform) its own quarter stays
#pragma unroll
                        for (int a = 0; a < A; ++a)
#pragma unroll
                            for (int c = 0; c < C; ++c) {
                                const int q = q0 + k;
                                red[((kw * QPR + k) * AC + a * C + c) * 64 + lane] =
                                    make_float4(acc[a][c][4 * q], acc[a][c][4 * q + 1],
                                                acc[a][c][4 * q + 2], acc[a][c][4 * q + 3]);
                            }
                    }
                    __syncthreads();
#pragma unroll
                    for (int k = 0; k < QPR; ++k) {
                        if (kw != q0 + k) continue;  // wave-uniform: here kw == q0 + k
#pragma unroll
                        for (int a = 0; a < A; ++a)
#pragma unroll
                            for (int c = 0; c < C; ++c) {
                                const int q = q0 + k;
                                const float4 *bp = red + (k * AC + a * C + c) * 64 + lane;
                                const int ws = QPR * AC * 64;  // one wave's words
                                const float4 own = make_float4(acc[a][c][4 * q], acc[a][c][4 * q + 1],
                                                               acc[a][c][4 * q + 2], acc[a][c][4 * q + 3]);
                                float4 v = q == 0 ? own : bp[0];
                                const float4 v1 = q == 1 ? own : bp[ws];
                                const float4 v2 = q == 2 ? own : bp[2 * ws];
                                const float4 v3 = q == 3 ? own : bp[3 * ws];
                                v.x += v1.x;
                                v.y += v1.y;
                                v.z += v1.z;
                                v.w += v1.w;
                                v.x += v2.x;
                                v.y += v2.y;
                                v.z += v2.z;
                                v.w += v2.w;
                                v.x += v3.x;
                                v.y += v3.y;
                                v.z += v3.z;
                                v.w += v3.w;
                                acc[a][c][0] = v.x;
                                acc[a][c][1] = v.y;
                                acc[a][c][2] = v.z;
                                acc[a][c][3] = v.w;
                            }
                    }
                }
                if constexpr (EPI == EPI_HEADNR && FH == 1) {
                    static_assert(A == 2 && C == 4, "64-value heads: two tiles by 128 tokens");
                    head_norm_rope64<T, C>(p, bd, acc, kw, h, r, m_blk, n_wave, (float *)lds_dyn);
                    return;
                } else if constexpr (EPI == EPI_HEADNR) {
                    float hv[2][4];
#pragma unroll
                    for (int a = 0; a < 2; ++a)
#pragma unroll
                        for (int e = 0; e < 4; ++e) hv[a][e] = acc[a][0][e];
                    // the scale/bias tables are no longer read (the reduction's
                    // first barrier follows every wave's last stage)
                    head_norm_rope<T>(p, bd, hv, hsn, hcs, fh, kw, h, r, m_blk,
                                      n_wave - 32 * fh, (float *)lds_dyn);
                    return;
                }
                const int blk = kw;  // this wave's quarter
                if constexpr (KM == KM_PART) {
                    float *dst = p.part + (int64_t)kz * p.M * bd.Nout;
#pragma unroll
                    for (int c = 0; c < C; ++c) {
                        const int64_t m = m_blk + 32 * c + r;
#pragma unroll
                        for (int a = 0; a < A; ++a) {
                            const int64_t n = n_wave + 32 * a + 8 * blk + 4 * h;
                            if (m < p.M && n < bd.Nout)
                                *(float4 *)(dst + m * bd.Nout + n) =
                                    make_float4(acc[a][c][0], acc[a][c][1], acc[a][c][2],
                                                acc[a][c][3]);
                        }
                    }
                } else {
                    // EPI_RESID: every residual load of the quarter first
                    uint2 rres[EPI == EPI_RESID ? C : 1][EPI == EPI_RESID ? A : 1];
                    if constexpr (EPI == EPI_RESID && P == 1) {
#pragma unroll
                        for (int c = 0; c < C; ++c)
#pragma unroll
                            for (int a = 0; a < A; ++a)
                                rres[c][a] = resid4<T>(p, bd, m_blk + 32 * c + r,
                                                       n_wave + 32 * a + 8 * blk + 4 * h);
                    }
#pragma unroll
                    for (int c = 0; c < C; ++c) {
                        const int64_t m = m_blk + 32 * c + r;
                        if constexpr (P == 1) {
#pragma unroll
                            for (int a = 0; a < A; ++a) {
                                float v[1][4] = {{acc[a][c][0], acc[a][c][1], acc[a][c][2],
                                                  acc[a][c][3]}};
                                const uint2 *rp = nullptr;
                                if constexpr (EPI == EPI_RESID) rp = &rres[c][a];
                                epi4<T, EPI, 1>(p, bd, m, n_wave + 32 * a + 8 * blk + 4 * h, v, rp);
                            }
                        } else {
                            float v[P][4];
#pragma unroll
                            for (int q = 0; q < P; ++q)
#pragma unroll
                                for (int e = 0; e < 4; ++e) v[q][e] = acc[q][c][e];
                            epi4<T, EPI, P>(p, bd, m, n_wave + 8 * blk + 4 * h, v);
                        }
                    }
                }
                return;
            }
        }

        if constexpr (Sh::KG > 1) {
            // Fixed-order reduction of the K-split partial tiles: K-group 0 adds
            // groups 1, 2, ... in turn. The ring's LDS is reused, RSLOTS partials
            // per round, so every wave must be done with its x stages first; all
            // waves take part in every round's barriers.
            constexpr int REGS = A * C * 16;
            float *red = (float *)lds;
            __syncthreads();
            for (int r0 = 1; r0 < wk; r0 += Sh::RSLOTS) {  // workgroup-uniform
                const int r1 = r0 + Sh::RSLOTS < wk ? r0 + Sh::RSLOTS : wk;
                if (kw >= r0 && kw < r1) {
                    float *dst = red + (size_t)(kw - r0) * REGS * 64 + lane;
#pragma unroll
                    for (int a = 0; a < A; ++a)
#pragma unroll
                        for (int c = 0; c < C; ++c)
#pragma unroll
                            for (int i = 0; i < 16; ++i) dst[((a * C + c) * 16 + i) * 64] = acc[a][c][i];
                }
                __syncthreads();
                if (kw == 0) {
                    for (int src = r0; src < r1; ++src) {
                        const float *sp = red + (size_t)(src - r0) * REGS * 64 + lane;
#pragma unroll
                        for (int a = 0; a < A; ++a)
#pragma unroll
                            for (int c = 0; c < C; ++c)
#pragma unroll
                                for (int i = 0; i < 16; ++i) acc[a][c][i] += sp[((a * C + c) * 16 + i) * 64];
                    }
                }
                if (r1 < wk) __syncthreads();  // the slots are refilled next round
            }
        }
        if constexpr (KM == KM_LOOP) {
            // wave 0 folds the part into the running sums, in part order; the
            // barrier keeps the next part's DMAs off the slots until it has read
            // the other waves' partials
            if (kw == 0) {
#pragma unroll
                for (int a = 0; a < A; ++a)
#pragma unroll
                    for (int c = 0; c < C; ++c)
#pragma unroll
                        for (int i = 0; i < 16; ++i) {
                            float *sp = psum + ((a * C + c) * 16 + i) * 64 + lane;
                            *sp = kp == 0 ? acc[a][c][i] : *sp + acc[a][c][i];
                        }
            }
            __syncthreads();
        }
    }  // K parts
    if (kw > 0) return;
    if constexpr (KM == KM_LOOP) {
#pragma unroll
        for (int a = 0; a < A; ++a)
#pragma unroll
            for (int c = 0; c < C; ++c)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[a][c][i] = psum[((a * C + c) * 16 + i) * 64 + lane];
    }
    if constexpr (KM == KM_PART) {
        // one K part's sums, fp32 [ks, M, Nout] (single-part epilogues; the
        // host checks Nout % 4 == 0): a second kernel adds the parts
        float *dst = p.part + (int64_t)kz * p.M * bd.Nout;
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const int64_t m = m_blk + 32 * c + r;
#pragma unroll
            for (int a = 0; a < A; ++a)
#pragma unroll
                for (int blk = 0; blk < 4; ++blk) {
                    const int64_t n = n_wave + 32 * a + 8 * blk + 4 * h;
                    if (m < p.M && n < bd.Nout)
                        *(float4 *)(dst + m * bd.Nout + n) =
                            make_float4(acc[a][c][4 * blk], acc[a][c][4 * blk + 1],
                                        acc[a][c][4 * blk + 2], acc[a][c][4 * blk + 3]);
                }
        }
        return;
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
                    epi4<T, EPI, 1>(p, bd, m, n_wave + 32 * a + 8 * blk + 4 * h, v);
                }
            } else {
                float v[P][4];
#pragma unroll
                for (int q = 0; q < P; ++q)
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[q][e] = acc[q][c][4 * blk + e];
                epi4<T, EPI, P>(p, bd, m, n_wave + 8 * blk + 4 * h, v);
            }
        }
    }
#endif  // __HIP_DEVICE_COMPILE__
}

template <typename T, int BITS, int A, int C, int WK, int EPI, int KM, bool KI = false>
__global__ __launch_bounds__(64 * WK)
__attribute__((amdgpu_waves_per_eu(mfma_waves_per_eu<A, C>()))) void qmm_mfma_kernel(
    QParams p) {
    constexpr int TN = (epi_parts(EPI) == 1) ? A : 1;
    __shared__ __attribute__((aligned(16))) char lds[MfmaShape<T, BITS, A, C, WK>::LDS];
    qmm_mfma_tile<T, BITS, A, C, WK, EPI, KM, 1, KI>(p, lds, (int64_t)blockIdx.x * (32 * TN),
                                                     (int64_t)blockIdx.y * (32 * C), (int)blockIdx.z);
}

// Block i of a run of n feature tiles that take g workgroups each (the g
// token blocks of a tile): tile j, token block part. A tile's workgroups sit 8
// blocks apart: blocks are dealt to MI355X's 8 XCDs in turn, so they land on
// one XCD and all but the first read the weight tile from its L2 (adjacent
// blocks fetched every weight byte g times from HBM). Groups of 8 tiles take
// 8 g blocks; a last partial group of r tiles spaces its blocks r apart.
__device__ __forceinline__ void mixed_tile_of(int i, int n, int g, int64_t &j, int64_t &part) {
    // 32-bit index math (grids are far below 2^31 blocks); g is 1, 2 or 4
    const int full = 8 * g * (n / 8);
    if (i < full) {
        j = 8 * (i / (8 * g)) + i % 8;
        part = (i / 8) % g;
    } else {
        const unsigned rem = (unsigned)(n % 8), t = (unsigned)(i - full);
        j = 8 * (n / 8) + t % rem;
        part = t / rem;
    }
}

// Mixed tiles for 64 < M <= 128, in two sizes: the first nb feature tiles
// take CB * 32-token tiles (128/(32 CB) workgroups each), the rest half that
// (twice the workgroups). With nb chosen so the grid is exactly two
// workgroups per CU, dealt so that no CU takes two of the larger ones, no CU
// runs one workgroup more than the others, which would finish a whole
// workgroup after the rest. Measured at M = 128:
// - the dual (CB = 4): 608 workgroups of 64 tokens took 32-33 us, against
//   25 us for 512; mixed, 29.6-30.3 us;
// - q/k/v (CB = 2): 384 workgroups of 64 tokens, 14.6-15.3 us; mixed with
//   32-token tiles, 13.2-13.3 us.
// Tiles never change the results (same K split and accumulation order).
template <typename T, int BITS, int A, int EPI, int CB>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(mfma_waves_per_eu<A, CB>()))) void qmm_mfma_mixed_kernel(
    QParams p) {
    static_assert(CB == 4 || CB == 2, "128/64- or 64/32-token tiles");
    constexpr int CS = CB / 2, GB = 4 / CB, GS = 2 * GB;
    constexpr int TN = (epi_parts(EPI) == 1) ? A : 1;
    constexpr int LB = MfmaShape<T, BITS, A, CB, 4>::LDS, LS = MfmaShape<T, BITS, A, CS, 4>::LDS;
    __shared__ __attribute__((aligned(16))) char lds[LB > LS ? LB : LS];
    const int64_t b = blockIdx.x, nb = p.n4;
    const int64_t nt = (p.Nout + 32 * TN - 1) / (32 * TN);
    int64_t j, part;
    if constexpr (CB == 4) {
        // (the 128-token tiles, one block each, written out directly: the
        // same mapping through mixed_tile_of ran the M = 128 dual at 33.8-34.0
        // instead of 29.5-29.7 us, A/B on one box, with an identical main
        // loop; the cause was not found)
        if (b < nb) {
            qmm_mfma_tile<T, BITS, A, CB, 4, EPI>(p, lds, b * (32 * TN), 0);
            return;
        }
    } else if (b < nb * GB) {
        mixed_tile_of((int)b, (int)nb, GB, j, part);
        qmm_mfma_tile<T, BITS, A, CB, 4, EPI>(p, lds, j * (32 * TN), part * 32 * CB);
        return;
    }
    mixed_tile_of((int)(b - nb * GB), (int)(nt - nb), GS, j, part);
    qmm_mfma_tile<T, BITS, A, CS, 4, EPI>(p, lds, (nb + j) * (32 * TN), part * 32 * CS);
}

// Three tile sizes for 64 < M <= 128 when the feature tiles outnumber the CUs
// by at most a quarter (cus < nt <= 5 cus / 4): a grid of exactly two
// workgroups per CU, block i and block cus + i sharing a CU. The first nb =
// 4 (nt - cus) feature tiles are 128-token tiles (blocks 0 .. nb - 1), each
// sharing its CU with a 32-token quarter of one of the last nb / 4 tiles
// (blocks cus .. cus + nb - 1, a tile's four quarters 8 blocks apart, on one
// XCD); the other tiles are 64-token pairs whose halves share a CU (blocks i
// and cus + i). Every CU then holds 160 or 128 tokens' worth of one feature
// tile's work, where the two-size grid left some CUs with 192 (a 128-token
// tile beside a 64-token one) and others with 128. The M = 128 dual (N =
// 9728, 256 CUs: 192 + 64 pairs + 48 quads) went 26.3-28.3 -> 24.3-25.5 us
// (A/B on one box), with the same bits.
template <typename T, int BITS, int A, int EPI>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(mfma_waves_per_eu<A, 4>()))) void qmm_mfma_mixed3_kernel(
    QParams p) {
    constexpr int TN = (epi_parts(EPI) == 1) ? A : 1;
    __shared__ __attribute__((aligned(16))) char lds[MfmaShape<T, BITS, A, 4, 4>::LDS];
    const int b = (int)blockIdx.x, nb = p.n4, cus = (int)(gridDim.x >> 1);
    if (b < nb) {  // 128-token tiles
        qmm_mfma_tile<T, BITS, A, 4, 4, EPI>(p, lds, (int64_t)b * (32 * TN), 0);
        return;
    }
    if (b < cus) {  // first halves of the pairs
        qmm_mfma_tile<T, BITS, A, 2, 4, EPI>(p, lds, (int64_t)b * (32 * TN), 0);
        return;
    }
    if (b < cus + nb) {  // quarters of the last nb / 4 tiles
        int64_t j, part;
        mixed_tile_of(b - cus, nb >> 2, 4, j, part);
        qmm_mfma_tile<T, BITS, A, 1, 4, EPI>(p, lds, (cus + j) * (32 * TN), part * 32);
        return;
    }
    // second halves of the pairs
    qmm_mfma_tile<T, BITS, A, 2, 4, EPI>(p, lds, (int64_t)(b - cus) * (32 * TN), 64);
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

// k values of the longest of the ks * wk wave chunks of K
inline int kslice_of(int64_t K, int ks, int wk) {
    return (int)ceil_div(K / XK, (int64_t)ks * wk) * XK;
}

// The interleaved K split: from M = 512 (a function of M and K only, so every
// tile shape at one (M, K) adds in the same order), one K part, four waves,
// while one scale/bias table over all of K fits the index multiplier of
// set_table (K / gs up to 358). The four waves then read adjacent stages
// (the 32-byte pieces of one 128-byte line of each weight row) at a time:
// LFM2's 2048-token prefill 6.30 -> 6.15 ms; at M = 128 the contiguous
// chunks keep more lines in flight per row and were the faster.
constexpr int64_t KINT_MIN_M = 512;
inline bool kint_of(const QParams &p, int wk) {
    if (p.M < KINT_MIN_M || p.ks != 1 || wk != 4) return false;
    const SbtLayout tl = sbt_layout(p.K, p.gs);
    return 8ll * tl.pitch * tl.pitch < (1ll << 20);
}
// k values one scale/bias table covers, and the tables of a workgroup
inline int table_kslice(const QParams &p, int wk) {
    return kint_of(p, wk) ? (int)p.K : kslice_of(p.K, p.ks, wk);
}
inline int table_count(const QParams &p, int wk) { return kint_of(p, wk) ? 1 : wk; }

// Running sums over the K parts (a workgroup that runs them in turn): one
// fp32 per accumulator register and lane.
inline int64_t mfma_sum_bytes(const QParams &p, int A, int C) {
    return (p.ks > 1 && !p.part) ? (int64_t)A * C * 16 * 64 * 4 : 0;
}

// Dynamic LDS of one workgroup: the waves' scale/bias tables and the sums
// over the K parts.
// (a table too long for the index multiplier of set_table counts as not
// fitting, so the dispatcher takes another kernel)
inline int64_t mfma_dyn_bytes(const QParams &p, int A, int C, int wk) {
    const SbtLayout tl = sbt_layout(table_kslice(p, wk), p.gs);
    if (8ll * tl.pitch * tl.pitch >= (1ll << 20)) return 1ll << 40;
    return (int64_t)table_count(p, wk) * A * 2 * tl.array_bytes + mfma_sum_bytes(p, A, C);
}

// LDS of one workgroup: the static stage slots plus the dynamic part.
template <typename T, int BITS, int A, int C>
int64_t mfma_lds_bytes(const QParams &p, int wk) {
    return MfmaShape<T, BITS, A, C, 4>::LDS + mfma_dyn_bytes(p, A, C, wk);
}

// The scale/bias table fields of p for wk waves: the longest chunk, the
// table layout, and the multiplier that divides a table dword index by
// pitch / 2 (exact for indices below 16 pitch while 8 pitch^2 < 2^20, i.e.
// K slices up to 360 groups; the host refuses longer ones).
inline bool set_table(QParams &p, int wk) {
    p.kint = kint_of(p, wk) ? 1 : 0;
    p.kslice = table_kslice(p, wk);
    const SbtLayout tl = sbt_layout(p.kslice, p.gs);
    p.sbp = tl.pitch;
    p.sbninst = tl.ninst;
    const unsigned half = (unsigned)(tl.pitch / 2);
    p.sbmagic = ((1u << 20) + half - 1) / half;
    return 8ll * tl.pitch * tl.pitch < (1ll << 20);
}

// p.ks K parts in grid z when p.part is set, else each workgroup runs them.
template <typename T, int BITS, int A, int C, int EPI, int KM = KM_ONE>
int launch_mfma_cfg(QParams p, int wk, hipStream_t st) {
    constexpr int P = epi_parts(EPI);
    constexpr int TN = (P == 1) ? A : 1;
    p.wk = wk;
    set_table(p, wk);
    const size_t dyn = (size_t)mfma_dyn_bytes(p, A, C, wk);
    if (mfma_lds_bytes<T, BITS, A, C>(p, wk) > LDS_PER_CU)
        return fail(MI_ERR_UNSUPPORTED, "quantized matmul tile exceeds the LDS (K = %lld)",
                    (long long)p.K);
    const dim3 grid((unsigned)ceil_div(p.Nout, 32 * TN), (unsigned)ceil_div(p.M, 32 * C),
                    p.part ? (unsigned)p.ks : 1u);
    if constexpr (KM == KM_ONE) {
        if (p.kint) {
            qmm_mfma_kernel<T, BITS, A, C, 4, EPI, KM, true><<<grid, 64 * wk, dyn, st>>>(p);
            return launch_status("quantized matmul (mfma)");
        }
    }
    qmm_mfma_kernel<T, BITS, A, C, 4, EPI, KM><<<grid, 64 * wk, dyn, st>>>(p);
    return launch_status("quantized matmul (mfma)");
}

// Compute units of the current device (cached per device).
int device_cus() {
    static int cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cache[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cache[dev] = n;
    }
    return cache[dev];
}

// qmm_mfma_mixed_kernel over nt feature tiles, the first nb of them as
// CB * 32-token tiles (four K-split waves).
template <typename T, int BITS, int A, int EPI, int CB>
int launch_mfma_mixed(QParams p, int nb, int64_t nt, hipStream_t st) {
    p.wk = 4;
    set_table(p, 4);
    p.n4 = nb;
    const size_t dyn = (size_t)mfma_dyn_bytes(p, A, CB, 4);
    const unsigned blocks = (unsigned)(nb * (4 / CB) + (nt - nb) * (8 / CB));
    qmm_mfma_mixed_kernel<T, BITS, A, EPI, CB><<<blocks, 256, dyn, st>>>(p);
    return launch_status("quantized matmul (mfma, mixed tiles)");
}

// qmm_mfma_mixed3_kernel: 2 cus blocks, the first nb = 4 (nt - cus) feature
// tiles as 128-token tiles.
template <typename T, int BITS, int A, int EPI>
int launch_mfma_mixed3(QParams p, int nb, int cus, hipStream_t st) {
    p.wk = 4;
    set_table(p, 4);
    p.n4 = nb;
    const size_t dyn = (size_t)mfma_dyn_bytes(p, A, 4, 4);
    qmm_mfma_mixed3_kernel<T, BITS, A, EPI><<<(unsigned)(2 * cus), 256, dyn, st>>>(p);
    return launch_status("quantized matmul (mfma, three tile sizes)");
}

// Tile choice (measured on MI355X over the Qwen3 prefill shapes, M = 128): one
// 32-feature tile per part (A = P) and 64-token tiles (C = 2) -- the smallest
// tiles that still reuse each x fragment across two MFMA columns -- give the
// most workgroups for these narrow-N GEMMs; 32-token tiles when 64-token tiles
// would leave fewer than 128 workgroups (half the CUs). From M = 512 (or past
// 2048 workgroups) 128-token tiles, two 32-feature tiles per wave for
// single-part outputs: re-reading x per narrow tile then costs more than the
// lost parallelism (LFM2 at M = 2048: down_proj 198 -> 99 us, out_proj 42 ->
// 30 us, the gate/up dual 257 -> 234 us). Tiles never change the numerics:
// the K split (wk) and each output's accumulation order are fixed by K.
// K must split into wk slices of whole 64-value x stages. A tile whose rings
// and scale/bias tables (which grow with K) exceed the LDS steps down to the
// next smaller one, and past the smallest the GEMV kernel runs instead.
template <typename T, int BITS, int EPI>
int launch_mfma(const QParams &p, hipStream_t st) {
    constexpr int P = epi_parts(EPI);
    // four K-split waves (chunks of whole stages, as even as the stage count
    // allows; one-part tiles reduce them across the four waves)
    const int wk = 4;
    // Several K parts without a workspace: each workgroup runs them in turn,
    // on 32-token tiles (the _ws entries run them as workgroups of their own)
    if (p.ks > 1) {
        if (mfma_lds_bytes<T, BITS, P, 1>(p, wk) <= LDS_PER_CU)
            return launch_mfma_cfg<T, BITS, P, 1, EPI, KM_LOOP>(p, wk, st);
        return launch_qmv<T, BITS, EPI>(p, st);
    }
    const int64_t nt = ceil_div(p.Nout, 32);
    const bool large = p.M >= 512 || nt * ceil_div(p.M, 64) > 2048;
    if constexpr (P == 1) {
        // (both widths. 8-bit took 32x128 tiles while its 64x128 tile
        // spilled; without the spill, LFM2's 8-bit out/down_proj at M = 2048
        // went 84.9 -> 64.4 us on average. The grouped q/k/v epilogue binds
        // one part per tile, so it takes 64-feature tiles only when every
        // part is a multiple of 64: LFM2's q/k/v at M = 2048, 6.35 -> 6.30 ms
        // a prefill against 32-feature tiles)
        const bool al2 = EPI != EPI_GROUP3 ||
                         (p.pn[0] % 64 == 0 && p.pn[1] % 64 == 0 && p.pn[2] % 64 == 0);
        // wide single-part 4-bit outputs take 64x128 tiles from M = 128
        // (N = 9728: 23.1 -> 21.3 us; narrower N loses parallelism)
        const bool wide = EPI != EPI_GROUP3 && p.M >= 128 && nt >= 256;
        if ((large || wide) && al2 && mfma_lds_bytes<T, BITS, 2, 4>(p, wk) <= LDS_PER_CU)
            return launch_mfma_cfg<T, BITS, 2, 4, EPI>(p, wk, st);
        if constexpr (EPI == EPI_GROUP3) {
            if (large && mfma_lds_bytes<T, BITS, 1, 4>(p, wk) <= LDS_PER_CU)
                return launch_mfma_cfg<T, BITS, 1, 4, EPI>(p, wk, st);
        }
    }
    if constexpr (P == 2) {
        if (large && mfma_lds_bytes<T, BITS, 2, 4>(p, wk) <= LDS_PER_CU)
            return launch_mfma_cfg<T, BITS, 2, 4, EPI>(p, wk, st);
    }
    // 64 < M <= 128 whose 64-token grid (2 nt workgroups) puts one workgroup
    // more on some CUs than on others: mixed tiles make it exactly two per CU,
    // at most one of the larger workgroups on each, when two of them fit a
    // CU's LDS (4-bit; measured only on the 4-bit Qwen3 shapes).
    // - more than two per CU (dual outputs): 128/64/32-token tiles while the
    //   feature tiles outnumber the CUs by at most a quarter, else 128/64;
    // - between one and one and a half per CU: 64/32-token tiles.
    // Aiming at one per CU does not pay: q/k/v at M = 128 with 128/64-token
    // tiles, 384 -> 256 workgroups, went 15.2 -> 15.4 us; a lone larger
    // workgroup takes as long as two smaller ones sharing a CU.
    if constexpr (BITS == 4 && P <= 2) {
        const int64_t cus = device_cus();
        if (p.M > 64 && p.M <= 128) {
            if constexpr (P == 2) {
                // up to a quarter more feature tiles than CUs: three sizes
                // (every workgroup allocates the 128-token tile's LDS)
                const int64_t nq = nt - cus;  // tiles cut into 32-token quarters
                if (nq > 0 && 4 * nq <= cus && cus % 8 == 0 &&
                    2 * mfma_lds_bytes<T, BITS, P, 4>(p, wk) <= LDS_PER_CU)
                    return launch_mfma_mixed3<T, BITS, P, EPI>(p, (int)(4 * nq), (int)cus, st);
                const int64_t nb4 = 2 * nt - 2 * cus;  // 128-token tiles
                if (nb4 > 0 && nb4 <= cus && 2 * mfma_lds_bytes<T, BITS, P, 4>(p, wk) <= LDS_PER_CU)
                    return launch_mfma_mixed<T, BITS, P, EPI, 4>(p, (int)nb4, nt, st);
            }
            const int64_t nb2 = 2 * nt - cus;  // 64-token tiles (two blocks each)
            if (nb2 > 0 && 2 * nb2 <= cus && 2 * mfma_lds_bytes<T, BITS, P, 2>(p, wk) <= LDS_PER_CU)
                return launch_mfma_mixed<T, BITS, P, EPI, 2>(p, (int)nb2, nt, st);
        }
    }
    if (p.M > 32 && nt * ceil_div(p.M, 64) >= 128 &&
        mfma_lds_bytes<T, BITS, P, 2>(p, wk) <= LDS_PER_CU) {
        // 32-token tiles instead when the 64-token tile's LDS (its scale/bias
        // tables grow with K) leaves fewer than three workgroups per CU and
        // the 32-token tile's does not (down_proj, K = 9728: 25.4 -> 23.2 us)
        const bool c1 = 3 * mfma_lds_bytes<T, BITS, P, 2>(p, wk) > LDS_PER_CU &&
                        3 * mfma_lds_bytes<T, BITS, P, 1>(p, wk) <= LDS_PER_CU;
        if (!c1) return launch_mfma_cfg<T, BITS, P, 2, EPI>(p, wk, st);
    }
    if (mfma_lds_bytes<T, BITS, P, 1>(p, wk) <= LDS_PER_CU)
        return launch_mfma_cfg<T, BITS, P, 1, EPI>(p, wk, st);
    return launch_qmv<T, BITS, EPI>(p, st);
}

template <typename T, int EPI>
int launch_qmv_dot2(const QParams &p, int mr, hipStream_t st) {
    // weights requested under the x staging when the 4-wave grid is at most
    // four workgroups per CU (measured: N = 9728 gains, N = 151936 loses),
    // for single-output epilogues: holding two or three weight rows' batches
    // through the staging takes 226-256 registers, one or two waves a SIMD
    // (the gate/up dual at M = 1, N = 9728: 10.9 us with PF, 8.6 without)
    const int64_t gy = ceil_div(p.M, mr);
    const bool pf = epi_parts(EPI) == 1 && mr == 1 && ceil_div(p.Nout, 16) * gy <= 1024 &&
                    p.K / 8 <= 512;
    // A row a wave (LPR 64) for single-output launches over long rows (K >
    // 4096, more than 8 chunks a lane at 16 lanes a row). Waves per workgroup
    // without PF: as many as spread the rows evenly over the CUs in one round
    // of workgroups (N = 9728 at 4 rows a wave: 10 waves, 244 workgroups, at
    // most 40 rows a CU, where 16-row workgroups put 48 on some CUs and 32 on
    // the others: M = 2 7.5 -> 7.2 us, M = 4 11.0 -> 9.6); 4 when the rows
    // take more than one round of 16-wave workgroups, for the grouped q/k/v
    // epilogue, whose workgroups each lie inside one part, and for the
    // several-output ones.
    constexpr bool wide_ok = qmv_dot2_wide_ok(EPI);
    const bool row_wave = wide_ok && !pf && p.K / 32 > 128;
    const int rpw = row_wave ? 1 : 4;
    int waves = 4;
    if constexpr (wide_ok) {
        const int64_t wv = ceil_div(p.Nout, rpw * (int64_t)device_cus());
        if (!pf && wv <= 16) waves = wv < 4 ? 4 : (int)wv;
    }
    const int bs = 64 * waves;
    const dim3 grid((unsigned)ceil_div(p.Nout, rpw * waves), (unsigned)gy);
    const size_t lds = (size_t)qmv_dot2_lds_bytes(mr, p.K);
    if (pf) {
        qmv_dot2_kernel<T, 1, EPI, true><<<grid, bs, lds, st>>>(p);
    } else if (!row_wave && waves == 4) {
        if (mr == 1)
            qmv_dot2_kernel<T, 1, EPI><<<grid, bs, lds, st>>>(p);
        else if (mr == 2)
            qmv_dot2_kernel<T, 2, EPI><<<grid, bs, lds, st>>>(p);
        else
            qmv_dot2_kernel<T, 4, EPI><<<grid, bs, lds, st>>>(p);
    } else if constexpr (wide_ok) {
        // a row a wave takes PF too at M = 1 while x fits two chunks a thread
        // (Qwen3's down_proj at decode, 10-wave workgroups: 6.7 -> 5.6 us)
        if (row_wave && mr == 1 && p.K / 8 <= 2 * bs) {
            if (waves == 4)
                qmv_dot2_kernel<T, 1, EPI, true, false, 64><<<grid, bs, lds, st>>>(p);
            else
                qmv_dot2_kernel<T, 1, EPI, true, true, 64><<<grid, bs, lds, st>>>(p);
        } else if (row_wave && waves == 4) {
            if (mr == 1)
                qmv_dot2_kernel<T, 1, EPI, false, false, 64><<<grid, bs, lds, st>>>(p);
            else if (mr == 2)
                qmv_dot2_kernel<T, 2, EPI, false, false, 64><<<grid, bs, lds, st>>>(p);
            else
                qmv_dot2_kernel<T, 4, EPI, false, false, 64><<<grid, bs, lds, st>>>(p);
        } else if (row_wave) {
            if (mr == 1)
                qmv_dot2_kernel<T, 1, EPI, false, true, 64><<<grid, bs, lds, st>>>(p);
            else if (mr == 2)
                qmv_dot2_kernel<T, 2, EPI, false, true, 64><<<grid, bs, lds, st>>>(p);
            else
                qmv_dot2_kernel<T, 4, EPI, false, true, 64><<<grid, bs, lds, st>>>(p);
        } else {
            if (mr == 1)
                qmv_dot2_kernel<T, 1, EPI, false, true><<<grid, bs, lds, st>>>(p);
            else if (mr == 2)
                qmv_dot2_kernel<T, 2, EPI, false, true><<<grid, bs, lds, st>>>(p);
            else
                qmv_dot2_kernel<T, 4, EPI, false, true><<<grid, bs, lds, st>>>(p);
        }
    }
    return launch_status("quantized matmul (dot2 qmv)");
}

// Shapes the MFMA kernel takes (16-bit T): it addresses x and each weight
// array with 32-bit offsets and copies scale/bias pairs with 4-byte loads (an
// even group count). wrows: rows of the largest part's arrays.
inline bool mfma_shape_ok(int64_t M, int64_t K, int64_t wrows, int gs, int bits) {
    return M > QMV_MR && K % XK == 0 && (K / gs) % 2 == 0 && M * K < ((int64_t)1 << 31) &&
           wrows * K * bits / 8 < ((int64_t)1 << 32);
}

template <typename T, int EPI>
int launch_typed(const QParams &p, int bits, hipStream_t st) {
    const bool mfma = (sizeof(T) == 2) && mfma_shape_ok(p.M, p.K, p.noff[2] + p.Nout, p.gs, bits);
    if constexpr (sizeof(T) == 2) {
        const int mr = p.M == 1 ? 1 : (p.M == 2 ? 2 : 4);
        if (bits == 4 && p.M <= 4 && qmv_dot2_lds_bytes(mr, p.K) <= 65536)
            return launch_qmv_dot2<T, EPI>(p, mr, st);
        if (mfma) {
            QParams q = p;
            q.ks = kpart_count(p.M, p.K);
            q.part = nullptr;
            return bits == 4 ? launch_mfma<T, 4, EPI>(q, st) : launch_mfma<T, 8, EPI>(q, st);
        }
    }
    return bits == 4 ? launch_qmv<T, 4, EPI>(p, st) : launch_qmv<T, 8, EPI>(p, st);
}

// The K-part launch (p.part set): 128-token tiles when M > 64, so a part
// dequantizes each weight once, and 64-feature tiles (4-bit) while they still
// make 128 workgroups. Single-part epilogues only; the parts kernel stores
// sums, and the epilogue runs in the kernel that adds them.
template <typename T, int BITS>
int launch_parts(const QParams &p, hipStream_t st) {
    const int wk = 4;
    const int C = p.M > 64 ? 4 : (p.M > 32 ? 2 : 1);
    const bool a2 = ceil_div(p.Nout, 64) * ceil_div(p.M, 32 * C) * p.ks >= 128;
    if constexpr (BITS == 4) {  // (the 8-bit 64x128 tile spills)
        if (a2 && C == 4 && mfma_lds_bytes<T, BITS, 2, 4>(p, wk) <= LDS_PER_CU)
            return launch_mfma_cfg<T, BITS, 2, 4, EPI_STORE, KM_PART>(p, wk, st);
        if (a2 && C == 2) return launch_mfma_cfg<T, BITS, 2, 2, EPI_STORE, KM_PART>(p, wk, st);
    }
    if (C == 4) return launch_mfma_cfg<T, BITS, 1, 4, EPI_STORE, KM_PART>(p, wk, st);
    if (C == 2) return launch_mfma_cfg<T, BITS, 1, 2, EPI_STORE, KM_PART>(p, wk, st);
    return launch_mfma_cfg<T, BITS, 1, 1, EPI_STORE, KM_PART>(p, wk, st);
}

// Adds the KS K parts of p.part in part order and applies the single-part
// epilogue EPI (EPI_STORE or EPI_RESID); thread t owns outputs 4t .. 4t + 3
// (Nout % 4 == 0, so a thread's four outputs lie in one row). Every load (the
// parts and the residual) is issued before the first add: a loop over a
// run-time part count had waited for each part's loads in turn.
template <typename T, int EPI, int KS>
__global__ __launch_bounds__(256) void qmm_parts_sum_kernel(QParams p) {
    static_assert(EPI == EPI_STORE || EPI == EPI_RESID, "single-part epilogues");
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t size = p.M * p.Nout;
    if (4 * q >= size) return;
    const int64_t o = 4 * q;
    float4 v[KS];
#pragma unroll
    for (int z = 0; z < KS; ++z) v[z] = *(const float4 *)(p.part + z * size + o);
    uint2 rr = {0, 0};
    if constexpr (EPI == EPI_RESID) rr = ld8((const T *)p.resid + o);
    float s[4] = {v[0].x, v[0].y, v[0].z, v[0].w};
#pragma unroll
    for (int z = 1; z < KS; ++z) {
        s[0] += v[z].x;
        s[1] += v[z].y;
        s[2] += v[z].z;
        s[3] += v[z].w;
    }
    // the [qmm] / [qmm, add] epilogue of epi4 on a whole 4-output group
    float y[4];
    if constexpr (EPI == EPI_RESID) {
        typedef typename Vec<T>::x4 V4;
        const V4 rv = __builtin_bit_cast(V4, rr);
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = pin32<T>((float)rv[e] + (float)cvt<T>(s[e]));
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = s[e];
    }
    st8((T *)p.y0 + o, pack4<T>(y));
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
    p.gs_log2 = ilog2(gs);
    p.wk = 1;
    p.ks = 1;
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

int64_t qmm_parts_bytes(int64_t M, int64_t N, int64_t K, int gs, int bits, int dtype) {
    if (dtype != MI_BF16 && dtype != MI_F16) return 0;
    if ((bits != 4 && bits != 8) || (gs != 32 && gs != 64 && gs != 128) || M < 0 || N <= 0)
        return 0;
    const int ks = kpart_count(M, K);
    if (ks < 2 || N % 4 || !mfma_shape_ok(M, K, N, gs, bits) || M * N >= ((int64_t)1 << 31))
        return 0;
    const int pitch = sbt_layout(kslice_of(K, ks, 4), gs).pitch;
    if (8ll * pitch * pitch >= (1ll << 20)) return 0;  // (the one-launch path takes it)
    // the narrowest tile launch_parts falls back to (one 32-feature tile a
    // wave at its token width) must fit the LDS, else the one-launch path
    // runs the shape (its dispatcher steps down tiles, then to the GEMV)
    QParams q = {};
    q.K = K;
    q.gs = gs;
    q.ks = ks;
    q.part = (float *)16;  // K parts as workgroups: no running sums in LDS
    const int64_t lds = M > 64 ? (bits == 4 ? mfma_lds_bytes<bf16, 4, 1, 4>(q, 4)
                                            : mfma_lds_bytes<bf16, 8, 1, 4>(q, 4))
                      : M > 32 ? (bits == 4 ? mfma_lds_bytes<bf16, 4, 1, 2>(q, 4)
                                            : mfma_lds_bytes<bf16, 8, 1, 2>(q, 4))
                               : (bits == 4 ? mfma_lds_bytes<bf16, 4, 1, 1>(q, 4)
                                            : mfma_lds_bytes<bf16, 8, 1, 1>(q, 4));
    if (lds > LDS_PER_CU) return 0;
    return (int64_t)ks * M * N * (int64_t)sizeof(float);
}

int qmm_parts_launch(const void *x, const uint32_t *w, const void *s, const void *b, float *part,
                     int64_t M, int64_t N, int64_t K, int gs, int bits, int dtype, void *stream) {
    if (int e = check_common(x, w, s, b, part, M, N, K, gs, bits, dtype)) return e;
    QParams p = base_params(x, w, s, b, nullptr, M, N, K, gs);
    p.ks = kpart_count(M, K);
    p.part = part;
    hipStream_t st = as_stream(stream);
    if (dtype == MI_BF16)
        return bits == 4 ? launch_parts<bf16, 4>(p, st) : launch_parts<bf16, 8>(p, st);
    return bits == 4 ? launch_parts<f16, 4>(p, st) : launch_parts<f16, 8>(p, st);
}

namespace {

// The workspace entries: the K parts as workgroups of their own, then their
// sum with the epilogue; the one-launch path (same sums, same order) when the
// shape has one K part or the workspace is missing or short.
template <int EPI>
int run_ws(QParams p, int bits, int dtype, void *ws, int64_t ws_bytes, void *stream) {
    if (p.M == 0 || p.Nout == 0) return MI_OK;
    const int64_t need = qmm_parts_bytes(p.M, p.Nout, p.K, p.gs, bits, dtype);
    if (need == 0 || !ws || ws_bytes < need || !aligned(ws, 16))
        return run<EPI>(p, bits, dtype, stream);
    if (int e = qmm_parts_launch(p.x, p.w[0], p.s[0], p.b[0], (float *)ws, p.M, p.Nout, p.K, p.gs,
                                 bits, dtype, stream))
        return e;
    p.ks = kpart_count(p.M, p.K);
    p.part = (float *)ws;
    const unsigned blocks = (unsigned)ceil_div(p.M * p.Nout / 4, 256);
    hipStream_t st = as_stream(stream);
    if (p.ks == KPARTS && dtype == MI_BF16)
        qmm_parts_sum_kernel<bf16, EPI, KPARTS><<<blocks, 256, 0, st>>>(p);
    else if (p.ks == KPARTS)
        qmm_parts_sum_kernel<f16, EPI, KPARTS><<<blocks, 256, 0, st>>>(p);
    else
        return fail(MI_ERR_UNSUPPORTED, "%d K parts", p.ks);
    return launch_status("quantized matmul (sum of K parts)");
}

}  // namespace

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

extern "C" int64_t mi_qmm_workspace_bytes(int64_t M, int64_t N, int64_t K, int group_size,
                                          int bits, int dtype) {
    return qmm_parts_bytes(M, N, K, group_size, bits, dtype);
}

extern "C" int mi_qmm_affine_ws(const void *x, const uint32_t *w, const void *scales,
                                const void *biases, void *y, int64_t M, int64_t N, int64_t K,
                                int group_size, int bits, int dtype, void *workspace,
                                int64_t workspace_bytes, void *stream) {
    if (int e = check_common(x, w, scales, biases, y, M, N, K, group_size, bits, dtype)) return e;
    return run_ws<EPI_STORE>(base_params(x, w, scales, biases, y, M, N, K, group_size), bits,
                             dtype, workspace, workspace_bytes, stream);
}

extern "C" int mi_qmm_affine_residual_ws(const void *x, const uint32_t *w, const void *scales,
                                         const void *biases, const void *resid, void *y,
                                         int64_t M, int64_t N, int64_t K, int group_size,
                                         int bits, int dtype, void *workspace,
                                         int64_t workspace_bytes, void *stream) {
    if (int e = check_common(x, w, scales, biases, y, M, N, K, group_size, bits, dtype)) return e;
    if (M && N && !resid) return fail(MI_ERR_ARG, "null residual");
    if (!aligned(resid, 8)) return fail(MI_ERR_ARG, "residual must be 8-byte aligned");
    QParams p = base_params(x, w, scales, biases, y, M, N, K, group_size);
    p.resid = resid;
    return run_ws<EPI_RESID>(p, bits, dtype, workspace, workspace_bytes, stream);
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

extern "C" int mi_qmm_affine_grouped3(const void *x, const uint32_t *const w[3],
                                      const void *const scales[3], const void *const biases[3],
                                      void *const y[3], int64_t M, const int64_t N[3], int64_t K,
                                      int group_size, int bits, int dtype, void *stream) {
    if (!w || !scales || !biases || !y || !N) return fail(MI_ERR_ARG, "null array argument");
    int64_t total = 0;
    for (int i = 0; i < 3; ++i) {
        if (int e = check_common(x, w[i], scales[i], biases[i], y[i], M, N[i], K, group_size,
                                 bits, dtype))
            return e;
        // every tile width (16 GEMV rows, 32 MFMA features) must divide each part
        if (N[i] % 32)
            return fail(MI_ERR_ARG, "grouped qmm needs each N to be a multiple of 32, got %lld",
                        (long long)N[i]);
        total += N[i];
    }
    QParams p = base_params(x, w[0], scales[0], biases[0], y[0], M, total, K, group_size);
    for (int i = 0; i < 3; ++i) {
        p.w[i] = w[i];
        p.s[i] = scales[i];
        p.b[i] = biases[i];
        p.py[i] = y[i];
        p.pn[i] = N[i];
    }
    return run<EPI_GROUP3>(p, bits, dtype, stream);
}

namespace mi {
namespace {

// Whole-head tiles: 128 features by 32 tokens, eight waves (two feature
// halves of two 32-feature tiles, each split over four K chunks). At the
// Qwen3 prefill size (48 heads x 4 token tiles) a CU holds one workgroup:
// eight waves there, where four waves of four tiles each took 15.2 against
// 12.9 us for the q/k/v GEMM alone on the mixed grid.
template <typename T, int BITS>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void qmm_headnr_kernel(
    QParams p) {
    __shared__ __attribute__((aligned(16))) char lds[2 * MfmaShape<T, BITS, 2, 1, 4>::LDS];
    qmm_mfma_tile<T, BITS, 2, 1, 4, EPI_HEADNR, KM_ONE, 2>(p, lds, (int64_t)blockIdx.x * 128,
                                                          (int64_t)blockIdx.y * 32);
}

// 64-value heads: two 32-feature tiles by 128 tokens a wave, four K-split
// waves (the grouped q/k/v tile at M >= 512).
template <typename T, int BITS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void qmm_headnr64_kernel(
    QParams p) {
    __shared__ __attribute__((aligned(16))) char lds[MfmaShape<T, BITS, 2, 4, 4>::LDS];
    qmm_mfma_tile<T, BITS, 2, 4, 4, EPI_HEADNR, KM_ONE, 1, true>(p, lds, (int64_t)blockIdx.x * 64,
                                                       (int64_t)blockIdx.y * 128);
}

template <typename T, int BITS>
int launch_headnr64(QParams p, hipStream_t st) {
    p.wk = 4;
    // (the grouped q/k/v launch it stands for takes the interleaved split at
    // these sizes too; where that does not apply, it declines)
    if (!set_table(p, 4) || !p.kint)
        return fail(MI_ERR_UNSUPPORTED, "fused q/k/v: K = %lld too long for the scale/bias table",
                    (long long)p.K);
    // the scale/bias tables (one, shared, under the interleaved K split this
    // tile always runs at: M >= 512); the exchange (8 x 128 floats) reuses them
    int64_t dyn = table_count(p, 4) * 2 * 2 * (int64_t)sbt_layout(p.kslice, p.gs).array_bytes;
    dyn = dyn > 8 * 128 * 4 ? dyn : 8 * 128 * 4;
    if (MfmaShape<T, BITS, 2, 4, 4>::LDS + dyn > LDS_PER_CU)
        return fail(MI_ERR_UNSUPPORTED, "fused q/k/v tile LDS (K = %lld)", (long long)p.K);
    const dim3 grid((unsigned)(p.Nout / 64), (unsigned)ceil_div(p.M, 128));
    qmm_headnr64_kernel<T, BITS><<<grid, 256, (size_t)dyn, st>>>(p);
    return launch_status("quantized q/k/v + norm + rope");
}

template <typename T, int BITS>
int launch_headnr(QParams p, hipStream_t st) {
    p.wk = 4;
    // the eight waves' scale/bias tables, each laid out for a quarter of K
    if (!set_table(p, 4))
        return fail(MI_ERR_UNSUPPORTED, "fused q/k/v: K = %lld too long for the scale/bias table",
                    (long long)p.K);
    const int64_t dyn = 8 * 2 * 2 * (int64_t)sbt_layout(p.kslice, p.gs).array_bytes;
    if (2 * MfmaShape<T, BITS, 2, 1, 4>::LDS + dyn > LDS_PER_CU)
        return fail(MI_ERR_UNSUPPORTED, "fused q/k/v tile exceeds the LDS (K = %lld)",
                    (long long)p.K);
    const dim3 grid((unsigned)(p.Nout / 128), (unsigned)ceil_div(p.M, 32));
    qmm_headnr_kernel<T, BITS><<<grid, 512, (size_t)dyn, st>>>(p);
    return launch_status("quantized q/k/v + norm + rope");
}

}  // namespace
}  // namespace mi

extern "C" int mi_qmm_affine_qkv_norm_rope(
    const void *x, const uint32_t *const w[3], const void *const scales[3],
    const void *const biases[3], const void *q_norm, const void *k_norm, void *q_out,
    void *k_cache, void *v_cache, int64_t B, int64_t L, int64_t Hq, int64_t Hkv, int64_t D,
    int64_t K, int group_size, int bits, float eps, int rope_dims, int traditional, float base,
    float scale, int64_t offset, int64_t kv_cap, int64_t kv_pos, int dtype, void *stream) {
    if (!w || !scales || !biases) return fail(MI_ERR_ARG, "null array argument");
    if (B < 0 || L < 0 || Hq <= 0 || Hkv <= 0 || D <= 0)
        return fail(MI_ERR_ARG, "qkv shape B=%lld L=%lld Hq=%lld Hkv=%lld D=%lld", (long long)B,
                    (long long)L, (long long)Hq, (long long)Hkv, (long long)D);
    const int64_t M = B * L;
    const int64_t N[3] = {Hq * D, Hkv * D, Hkv * D};
    void *const y[3] = {q_out, k_cache, v_cache};
    for (int i = 0; i < 3; ++i)
        if (int e = check_common(x, w[i], scales[i], biases[i], y[i], M, N[i], K, group_size,
                                 bits, dtype))
            return e;
    if (kv_pos < 0 || kv_pos + L > kv_cap)
        return fail(MI_ERR_ARG, "rows [%lld, %lld) exceed the cache capacity %lld",
                    (long long)kv_pos, (long long)(kv_pos + L), (long long)kv_cap);
    if (!(base > 0.0f)) return fail(MI_ERR_ARG, "rope base must be positive");
    // The fused form covers 16-bit heads of 128 values up to M = 256 (past
    // that the grouped launch's larger tiles win: at 384 tokens the fused
    // launch took 34.9 against 33.7 us for the two launches, at 2048 134
    // against 98; at 160 15.9 against 21.5), or of 64 values from M = 512
    // (its 128-token tile; the grouped launch takes the same tile there),
    // rotated whole (not traditional), both norms, the MFMA path's shapes, and
    // 16-byte aligned norm weights and outputs (the layout under which the
    // separate launch takes the 16- or 8-lane form whose arithmetic the
    // epilogue repeats).
    const bool d128 = D == 128 && rope_dims == 128 && M <= 256;
    const bool d64 = D == 64 && rope_dims == 64 && M >= 512;
    if (dtype == MI_F32 || !(d128 || d64) || traditional || !q_norm || !k_norm)
        return fail(MI_ERR_UNSUPPORTED, "fused q/k/v + norm + rope covers 16-bit, D = rope dims "
                                        "= 128 up to M = 256 or 64 from M = 512, both norms");
    if (!mfma_shape_ok(M, K, N[0], group_size, bits) ||
        !mfma_shape_ok(M, K, N[1], group_size, bits))
        return fail(MI_ERR_UNSUPPORTED, "fused q/k/v + norm + rope: M=%lld K=%lld off the MFMA path",
                    (long long)M, (long long)K);
    if (!aligned(q_norm, 16) || !aligned(k_norm, 16) || !aligned(q_out, 16) ||
        !aligned(k_cache, 16) || !aligned(v_cache, 16))
        return fail(MI_ERR_UNSUPPORTED, "fused q/k/v + norm + rope needs 16-byte aligned rows");
    if (M == 0) return MI_OK;
    QParams p = base_params(x, w[0], scales[0], biases[0], q_out, M, N[0] + N[1] + N[2], K,
                            group_size);
    for (int i = 0; i < 3; ++i) {
        p.w[i] = w[i];
        p.s[i] = scales[i];
        p.b[i] = biases[i];
        p.py[i] = y[i];
        p.pn[i] = N[i];
    }
    p.nw[0] = q_norm;
    p.nw[1] = k_norm;
    p.L = L;
    p.cap = kv_cap;
    p.pos0 = kv_pos;
    p.offset = offset;
    p.eps = eps;
    p.log2base = (float)log2((double)base);
    p.rscale = scale;
    hipStream_t st = as_stream(stream);
    if (D == 64) {
        if (dtype == MI_BF16)
            return bits == 4 ? launch_headnr64<bf16, 4>(p, st) : launch_headnr64<bf16, 8>(p, st);
        return bits == 4 ? launch_headnr64<f16, 4>(p, st) : launch_headnr64<f16, 8>(p, st);
    }
    if (dtype == MI_BF16)
        return bits == 4 ? launch_headnr<bf16, 4>(p, st) : launch_headnr<bf16, 8>(p, st);
    return bits == 4 ? launch_headnr<f16, 4>(p, st) : launch_headnr<f16, 8>(p, st);
}
