// Row A7: causal GQA scaled-dot-product attention (mx.fast.scaled_dot_product_attention
// with mask='causal' or none), flash-style over 32-key tiles.
//
// The arithmetic of one query row is fixed: its key tiles of 32 (from key 0)
// are dealt to four streams by tile index (stream w: tiles w, w + 4, ...);
// each stream runs its own online softmax from scratch; the streams' states
// are then folded in stream order. Two kernels carry it out, bit for bit
// alike (same tile-update and merge functions, no floating-point
// contraction in them):
//   attn_split_kernel   one workgroup per (q head, 32-row q block); its four
//                       waves run the four streams side by side and merge in
//                       LDS. Many workgroups for short sequences (prefill of
//                       128: 128 workgroups) and for decode.
//   attn_shared_kernel  one workgroup per (kv head, 4 q heads, 32-row q
//                       block); its waves are the q heads of one GQA group
//                       (kv head of q head h is h / (H/HK),
//                       tests/test_graph_model_matrix.py:84-93) and share
//                       each K/V tile staged in LDS; each wave runs the
//                       streams one after another. A quarter of the K/V reads,
//                       for long sequences.
// The launcher picks by grid size; the choice never changes a result.
// Per wave and tile:
//   S^T[key][q] = K . Q^T   32x32x16 MFMA, A = K rows, B = Q^T held in
//                           registers for the whole kernel;
//   lane (q = lane%32, half) then holds 16 of the 32 keys of its query row, so
//   the row max/sum needs one xor-32 shuffle;
//   O^T[d][q] += V^T . P^T  A = V^T, read by transposing LDS loads from the
//                           V tile staged key-major as it sits in memory,
//                           B = P^T straight from the S^T registers
//                           (bf16/fp16): the k order inside each MFMA is
//                           permuted to match the S^T register layout, for
//                           both operands.
// Online softmax in the log2 domain, fp32 running max/sum, one division at
// the end. Causal masking is bottom-right aligned (query i sees keys
// j <= i + Lk - Lq) and key tiles past the last visible key are skipped.
// A row's result depends only on its global position and the keys, so a
// chunked prefill whose chunks start at multiples of 32 reproduces the whole
// prefill bit for bit.
#include <math.h>

#include "mi_common.h"

namespace mi {
namespace {

template <typename T> struct AMfma;
template <> struct AMfma<bf16> {
    static __device__ __forceinline__ f32x16 mma(bf16x8 a, bf16x8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};
template <> struct AMfma<f16> {
    static __device__ __forceinline__ f32x16 mma(f16x8 a, f16x8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

constexpr int ATT_KT = 32;       // keys per tile
constexpr int ATT_STREAMS = 4;   // key-tile streams per query row
// Row pitch (elements) of a key-major V tile in LDS: D + 16, so the four key
// rows one 16-lane group reads (32 bytes of each) start 8 banks apart.
template <int D> constexpr int att_vpitch() { return D + 16; }

// Online-softmax state of one wave: O^T tiles (lane = query column r, half
// h2), the row's reference maximum m (log2 units) and this lane's half of the
// row sum l.
template <int D> struct AttnState {
    f32x16 o[D / 32];
    float m, l;
};

template <int D> __device__ __forceinline__ void attn_init(AttnState<D> &st) {
#pragma unroll
    for (int t = 0; t < D / 32; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) st.o[t][i] = 0.0f;
    st.m = -INFINITY;
    st.l = 0.0f;
}

// One key tile kt, in two steps. attn_scores: s = S^T (s[i]: key
// kt*32 + 8*(i/4) + 4*h2 + i%4 of query row qrow) -> masking and the lazily
// rescaled online softmax; p gets the tile's probabilities. attn_pv:
// O^T += V^T . P^T, vs = the tile's V in LDS (32 key rows of att_vpitch<D>()
// elements). attn_tile runs both; the split kernel runs the scores before its
// V tile is written.
template <int D>
__device__ __forceinline__ void attn_scores(AttnState<D> &st, const f32x16 &s, float (&p)[16],
                                            int kt, int64_t q0, int64_t qrow, int64_t off,
                                            int64_t Lk, int causal, float scale_log2, int h2) {
#pragma clang fp contract(off)
    constexpr int DT = D / 32;
    float mt = -INFINITY;
    // a tile whose every key every row of the block sees needs no mask
    const bool full = (int64_t)kt * ATT_KT + ATT_KT <= Lk &&
                      (!causal || (int64_t)kt * ATT_KT + ATT_KT - 1 <= q0 + off);
    const int vis_end = (int)((causal && qrow + off + 1 < Lk ? qrow + off + 1 : Lk) -
                              (int64_t)kt * ATT_KT);  // keys [0, vis_end) of the tile
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int kl = 8 * (i / 4) + 4 * h2 + (i % 4);
        p[i] = (full || kl < vis_end) ? s[i] * scale_log2 : -INFINITY;
        mt = fmaxf(mt, p[i]);
    }
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    // Lazy rescale: the exponents are taken against a running reference m
    // that moves only when a row's maximum passes it by more than 8 (log2
    // units). p then stays below 2^8, where fp32 sums and the bf16/fp16 P
    // operand keep their relative precision, and the accumulator rescales run
    // only on those (wave-uniform) steps.
    const bool grow = mt > st.m + 8.0f;
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
        const float m_new = grow ? mt : st.m;
        const float corr = st.m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(st.m - m_new);
        st.l *= corr;
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) st.o[t][i] *= corr;
        st.m = m_new;
    }
    const bool none = st.m == -INFINITY;
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        p[i] = none ? 0.0f : __builtin_amdgcn_exp2f(p[i] - st.m);
        psum += p[i];
    }
    st.l += psum;
}

// Four 16-bit values by ds_read_b64_tr_b16. Within each 16-lane group, with
// lane s addressing four consecutive values E[s][0..3], lane 4a + b receives
// (E[a][b], E[a + 4][b], E[a + 8][b], E[a + 12][b]) (probed on gfx950: LDS
// filled with each value's index, lanes addressing rows of 4 and of 16).
template <typename T>
__device__ __forceinline__ typename Vec<T>::x4 lds_read_tr4(const T *p) {
    typedef short S4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) S4 *LP;
    return __builtin_bit_cast(typename Vec<T>::x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((LP)p));
}

// A fragment of O^T += V^T . P^T for lane (r, h2), MFMA k2 of head-dim tile
// t: V^T[32 t + r][keys 16 k2 + 4 h2 + (0..3), then the same + 8]. Lane s of
// 16-lane group G addresses key row 16 k2 + 4 h2 + s / 4 (h2 = G / 2) at
// column 32 t + 16 (G % 2) + 4 (s % 4); by the rule above lane 4a + b of the
// group (r = 16 (G % 2) + 4a + b) then receives column 32 t + r of the key
// rows 16 k2 + 4 h2 + 0..3.
template <typename T, int D>
__device__ __forceinline__ void attn_pv(AttnState<D> &st, const float (&p)[16], const T *vs,
                                        int lane) {
#pragma clang fp contract(off)
    constexpr int DT = D / 32, VP = att_vpitch<D>();
    typedef typename Vec<T>::x8 V8;
    typedef typename Vec<T>::x4 V4;
    const int s = lane & 15, g = lane >> 4;
    const T *vl = vs + (4 * (g >> 1) + (s >> 2)) * VP + 16 * (g & 1) + 4 * (s & 3);
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
        V8 pb;
#pragma unroll
        for (int e = 0; e < 8; ++e) pb[e] = (T)p[8 * k2 + e];
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            const T *vr = vl + 16 * k2 * VP + 32 * t;
            const V4 lo = lds_read_tr4<T>(vr);
            const V4 hi = lds_read_tr4<T>(vr + 8 * VP);
            V8 a;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                a[e] = lo[e];
                a[4 + e] = hi[e];
            }
            st.o[t] = AMfma<T>::mma(a, pb, st.o[t]);
        }
    }
}

template <typename T, int D>
__device__ __forceinline__ void attn_tile(AttnState<D> &st, const f32x16 &s, const T *vs, int kt,
                                          int64_t q0, int64_t qrow, int64_t off, int64_t Lk,
                                          int causal, float scale_log2, int h2, int lane) {
    float p[16];
    attn_scores<D>(st, s, p, kt, q0, qrow, off, Lk, causal, scale_log2, h2);
    attn_pv<T, D>(st, p, vs, lane);
}

// Folding a later stream's state (mw, lw, o_w) into a running (m, l, o):
// m' = max(m, mw); o' = o c0 + o_w cw and l' = l c0 + lw cw with
// c0 = 2^(m - m'), cw = 2^(mw - m'). A stream that saw no visible key of the
// row (mw = -inf) leaves the state as it is.
struct MergeCoef {
    float c0, cw, m_new;
};
__device__ __forceinline__ MergeCoef merge_coef(float m, float mw) {
#pragma clang fp contract(off)
    const float m_new = fmaxf(m, mw);
    return {m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - m_new),
            __builtin_amdgcn_exp2f(mw - m_new), m_new};
}
__device__ __forceinline__ float merge_one(float o, float ow, const MergeCoef &c) {
#pragma clang fp contract(off)
    return __builtin_fmaf(o, c.c0, ow * c.cw);
}

template <int D, typename OW>
__device__ __forceinline__ void attn_merge(AttnState<D> &st, float mw, float lw, OW ow) {
    if (mw == -INFINITY) return;
    const MergeCoef c = merge_coef(st.m, mw);
#pragma unroll
    for (int t = 0; t < D / 32; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) st.o[t][i] = merge_one(st.o[t][i], ow(t, i), c);
    st.l = merge_one(st.l, lw, c);
    st.m = c.m_new;
}

// Output tile t (features 32 t .. 32 t + 31) of the lane's query row: O^T / row sum.
template <typename T>
__device__ __forceinline__ void attn_store_tile(const f32x16 &o, float l, T *orow, int t, int h2) {
#pragma clang fp contract(off)
    const float l_tot = l + __shfl_xor(l, 32, 64);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
        float f[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = o[4 * blk + e] * inv;
        st8(orow + 32 * t + 8 * blk + 4 * h2, pack4<T>(f));
    }
}

template <typename T, int D>
__device__ __forceinline__ void attn_store(const AttnState<D> &st, T *orow, int h2) {
#pragma unroll
    for (int t = 0; t < D / 32; ++t) attn_store_tile<T>(st.o[t], st.l, orow, t, h2);
}

// Key tiles visible to a q block (causal: up to its last row).
__device__ __forceinline__ int attn_ntiles(int64_t q0, int64_t off, int64_t Lk, int causal) {
    int64_t kend = Lk;
    if (causal) {
        const int64_t last = q0 + 31 + off + 1;
        kend = last < Lk ? last : Lk;
    }
    return kend > 0 ? (int)ceil_div(kend, ATT_KT) : 0;
}

// ---------------------------------------------------------------------------
// attn_split_kernel: workgroup = (q head, q block); wave w runs stream w.

template <int D> struct SplitLds {
    static constexpr int DT = D / 32;
    static constexpr int VT_BYTES = ATT_KT * att_vpitch<D>() * 2;  // one wave's V tile
    static constexpr int PART_FLOATS = DT * 16 * 64 + 2 * 64;  // one wave's state
    static constexpr int BYTES = ATT_STREAMS * VT_BYTES > ATT_STREAMS * PART_FLOATS * 4
                                     ? ATT_STREAMS * VT_BYTES
                                     : ATT_STREAMS * PART_FLOATS * 4;
};

template <typename T, int D>
__global__ __launch_bounds__(64 * ATT_STREAMS) void attn_split_kernel(
    const T *__restrict__ q, const T *__restrict__ k, const T *__restrict__ v,
    T *__restrict__ out, int64_t H, int64_t HK, int64_t Lq, int64_t Lk, int64_t cap,
    float scale_log2, int causal, int out_layout) {
    typedef SplitLds<D> L;
    constexpr int DT = D / 32;
    constexpr int DS = D / 16;  // MFMA k-steps over the head dim
    typedef typename Vec<T>::x8 V8;
    __shared__ __attribute__((aligned(16))) char lds[L::BYTES];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h2 = lane >> 5, r = lane & 31;
    // block index -> (b, q head, q block) in 32-bit math (grids are far below
    // 2^31 blocks; 64-bit divisions cost hundreds of scalar instructions)
    unsigned bid = blockIdx.x;
    const unsigned nqb = (unsigned)ceil_div(Lq, 32);
    const int64_t qblk = bid % nqb;
    bid /= nqb;
    const int64_t hq = bid % (unsigned)H, b = bid / (unsigned)H;
    const int64_t hk = (unsigned)hq / (unsigned)(H / HK);
    const int64_t q0 = qblk * 32;
    const int64_t off = Lk - Lq;
    const int64_t qrow = q0 + r;
    const bool qok = qrow < Lq;

    // The q block (32 rows x D) is read once per workgroup: each thread loads
    // QPT of its 16-byte chunks (rows past Lq: zeros) and stores them to LDS,
    // 16-byte chunk c of row rr at position c ^ (rr % (D / 8)), so the 32 rows'
    // reads of one chunk hit distinct banks; after the barrier below every
    // wave reads its MFMA fragments. (Each wave had loaded the whole block.)
    constexpr int QCR = D / 8;         // 16-byte chunks per q row
    constexpr int QPT = 32 * QCR / 256;  // chunks per thread
    __shared__ uint4 qsh[32 * QCR];
    uint4 qv[QPT];
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
        const int c = (int)threadIdx.x + 256 * i, rr = c / QCR;
        qv[i] = q0 + rr < Lq ? ld16(q + ((b * H + hq) * Lq + q0 + rr) * D + 8 * (c % QCR))
                             : make_uint4(0, 0, 0, 0);
    }
    AttnState<D> st;
    attn_init(st);
    const int ntiles = attn_ntiles(q0, off, Lk, causal);
    const T *kb = k + (b * HK + hk) * cap * D;
    const T *vb = v + (b * HK + hk) * cap * D;
    T *vs = (T *)(lds + wave * L::VT_BYTES);  // this wave's V tile (key-major)

    // A tile's loads: the K rows as MFMA A fragments (key r, head-dim chunk
    // 16 s + 8 h2), and V as 16-byte chunks (key r, chunk h2 + 2 i) for the
    // key-major LDS tile. Keys past Lk read the last key (in bounds): their
    // scores are masked and their V rows zeroed.
    constexpr int VCH = D / 16;  // V chunks per lane
    uint4 kf[DS], vreg[VCH];
    auto fetch = [&](int kt) {
        const int64_t kg = (int64_t)kt * ATT_KT + r;
        const int64_t kc = kg < Lk ? kg : Lk - 1;
#pragma unroll
        for (int s = 0; s < DS; ++s) kf[s] = ld16(kb + kc * D + 16 * s + 8 * h2);
#pragma unroll
        for (int i = 0; i < VCH; ++i) vreg[i] = ld16(vb + kc * D + (h2 + 2 * i) * 8);
    };
    // every wave issues its first tile's loads (a wave past the last tile a
    // clamped, unused one), so the wait for q below leaves them in flight
    fetch(wave);
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
        const int c = (int)threadIdx.x + 256 * i, rr = c / QCR;
        qsh[rr * QCR + ((c % QCR) ^ (rr % QCR))] = qv[i];
    }
    __syncthreads();
    uint4 qf[DS];
#pragma unroll
    for (int s = 0; s < DS; ++s) qf[s] = qsh[r * QCR + ((2 * s + h2) ^ (r % QCR))];

    for (int kt = wave; kt < ntiles; kt += ATT_STREAMS) {  // wave-uniform
        // S^T and the softmax first: the V loads, issued after K's, land
        // under the MFMAs and the exponentials
        f32x16 s;
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < DS; ++ks)
            s = AMfma<T>::mma(__builtin_bit_cast(V8, kf[ks]), __builtin_bit_cast(V8, qf[ks]), s);
        float p[16];
        attn_scores<D>(st, s, p, kt, q0, qrow, off, Lk, causal, scale_log2, h2);
        // V tile: this wave's own LDS, written and read by this wave only
        // (its LDS instructions execute in order)
        const bool vok = (int64_t)kt * ATT_KT + r < Lk;
#pragma unroll
        for (int i = 0; i < VCH; ++i)
            *(uint4 *)(vs + r * att_vpitch<D>() + (h2 + 2 * i) * 8) =
                vok ? vreg[i] : make_uint4(0, 0, 0, 0);
        if (kt + ATT_STREAMS < ntiles) fetch(kt + ATT_STREAMS);  // under this tile's math
        attn_pv<T, D>(st, p, vs, lane);
    }

    // Merge: every wave leaves its stream's (o, l, m) in LDS (over the V
    // tiles) as 16-byte words; wave w then folds the four streams, in stream
    // order, for O^T tile t = w (D = 64: tiles 0 and 1) and stores that tile.
    // Each wave recomputes the same (m, l) chain, so the result is that of one
    // wave folding every tile.
    // Layout of a wave's state: float4 [DT * 4][64] (accumulator registers
    // 4j .. 4j + 3 of tile t at t * 4 + j), then float2 (l, m) [64].
    float4 *part = (float4 *)lds;
    constexpr int PART4 = L::PART_FLOATS / 4;  // one wave's state in float4
    __syncthreads();  // every wave is done with its V tile
    {
        float4 *pp = part + (size_t)wave * PART4;
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                pp[(t * 4 + j) * 64 + lane] = make_float4(st.o[t][4 * j], st.o[t][4 * j + 1],
                                                          st.o[t][4 * j + 2], st.o[t][4 * j + 3]);
        ((float2 *)(pp + DT * 4 * 64))[lane] = make_float2(st.l, st.m);
    }
    __syncthreads();
    if (!qok) return;
    T *orow = out_layout ? out + ((b * Lq + qrow) * H + hq) * D
                         : out + ((b * H + hq) * Lq + qrow) * D;
    for (int t = wave; t < DT; t += ATT_STREAMS) {  // wave-uniform
        f32x16 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4 v = part[(t * 4 + j) * 64 + lane];
            o[4 * j] = v.x;
            o[4 * j + 1] = v.y;
            o[4 * j + 2] = v.z;
            o[4 * j + 3] = v.w;
        }
        const float2 lm = ((const float2 *)(part + DT * 4 * 64))[lane];
        float l = lm.x, m = lm.y;
        for (int w = 1; w < ATT_STREAMS; ++w) {
            const float4 *pp = part + (size_t)w * PART4;
            const float2 lmw = ((const float2 *)(pp + DT * 4 * 64))[lane];
            const float mw = lmw.y;
            if (mw == -INFINITY) continue;
            const MergeCoef c = merge_coef(m, mw);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 v = pp[(t * 4 + j) * 64 + lane];
                o[4 * j] = merge_one(o[4 * j], v.x, c);
                o[4 * j + 1] = merge_one(o[4 * j + 1], v.y, c);
                o[4 * j + 2] = merge_one(o[4 * j + 2], v.z, c);
                o[4 * j + 3] = merge_one(o[4 * j + 3], v.w, c);
            }
            l = merge_one(l, lmw.x, c);
            m = c.m_new;
        }
        attn_store_tile<T>(o, l, orow, t, h2);
    }
}

// ---------------------------------------------------------------------------
// attn_shared_kernel: workgroup = (kv head, quad of its q heads, q block);
// the four waves share each K/V tile and run the streams in turn.

template <typename T, int D>
__global__ __launch_bounds__(256) void attn_shared_kernel(
    const T *__restrict__ q, const T *__restrict__ k, const T *__restrict__ v,
    T *__restrict__ out, int64_t H, int64_t HK, int64_t Lq, int64_t Lk, int64_t cap,
    float scale_log2, int causal, int out_layout, int quads, int zig) {
    constexpr int KP = D + 8;  // padded K-tile row (elements)
    constexpr int DS = D / 16;
    typedef typename Vec<T>::x8 V8;
    __shared__ __attribute__((aligned(16))) T ks[ATT_KT * KP];
    __shared__ __attribute__((aligned(16))) T vs[ATT_KT * att_vpitch<D>()];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h2 = lane >> 5, r = lane & 31;
    unsigned bid = blockIdx.x;  // 32-bit index math, as in attn_split_kernel
    const unsigned nqb = (unsigned)ceil_div(Lq, 32);
    int64_t qblk;
    if (zig) {
        // (nqb even) block b and b + G/2 take q blocks j and nqb - 1 - j of
        // the same heads: under causal masking their key-tile counts add up
        // to nqb + 1 for every pair, and a grid of two workgroups per CU
        // places b and b + G/2 on one CU
        const unsigned g2 = gridDim.x >> 1, hb = nqb >> 1;
        const unsigned second = bid >= g2, u = bid - (second ? g2 : 0u);
        const unsigned j = u % hb;
        qblk = second ? nqb - 1 - j : j;
        bid = u / hb;
    } else {
        qblk = bid % nqb;
        bid /= nqb;
    }
    const int quad = (int)(bid % (unsigned)quads);
    bid /= (unsigned)quads;
    const int64_t hk = bid % (unsigned)HK, b = bid / (unsigned)HK;
    const int64_t rep = H / HK;
    const bool active = quad * 4 + wave < rep;
    const int64_t hq = hk * rep + (active ? quad * 4 + wave : 0);
    const int64_t q0 = qblk * 32;
    const int64_t off = Lk - Lq;
    const int64_t qrow = q0 + r;
    const bool qok = active && qrow < Lq;

    uint4 qf[DS];
    {
        const T *qp = q + ((b * H + hq) * Lq + (qok ? qrow : 0)) * D + 8 * h2;
#pragma unroll
        for (int s = 0; s < DS; ++s) qf[s] = qok ? ld16(qp + 16 * s) : make_uint4(0, 0, 0, 0);
    }
    const int ntiles = attn_ntiles(q0, off, Lk, causal);
    const T *kb = k + (b * HK + hk) * cap * D;
    const T *vb = v + (b * HK + hk) * cap * D;

    // K/V tile staging: each thread owns CH 16-byte chunks of a tile; the
    // chunks of the next tile are loaded into registers while this one
    // computes. Both tiles are key-major in LDS (V is read transposed).
    constexpr int CH = ATT_KT * D / 8 / 256;
    uint4 kreg[CH], vreg[CH];
    auto fetch = [&](int kt) {
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int c = threadIdx.x + 256 * i;
            const int key = c % ATT_KT, dc = c / ATT_KT;
            const int64_t kg = (int64_t)kt * ATT_KT + key;
            const int64_t kc = kg < Lk ? kg : Lk - 1;  // in bounds; masked below
            kreg[i] = ld16(kb + kc * D + dc * 8);
            vreg[i] = ld16(vb + kc * D + dc * 8);
        }
    };
    // tiles in stream order: 0, 4, 8, ..., then 1, 5, 9, ..., and so on
    auto next_tile = [&](int kt) -> int {
        if (kt + ATT_STREAMS < ntiles) return kt + ATT_STREAMS;
        const int s = kt % ATT_STREAMS + 1;
        return s < ATT_STREAMS && s < ntiles ? s : -1;
    };
    // One pass per stream: its tiles in turn into cur, then cur folded into
    // tot in stream order. (With the fold inside one loop over all tiles the
    // compiler copied both states at every tile.)
    AttnState<D> tot;
    attn_init(tot);
    if (ntiles > 0) fetch(0);
    const int nstreams = ntiles < ATT_STREAMS ? ntiles : ATT_STREAMS;
    for (int sw = 0; sw < nstreams; ++sw) {  // workgroup-uniform
        AttnState<D> cur;
        attn_init(cur);
        for (int kt = sw; kt < ntiles; kt += ATT_STREAMS) {  // workgroup-uniform
            __syncthreads();  // every wave is done with the previous tile
#pragma unroll
            for (int i = 0; i < CH; ++i) {
                const int c = threadIdx.x + 256 * i;
                const int key = c % ATT_KT, dc = c / ATT_KT;
                const bool ok = (int64_t)kt * ATT_KT + key < Lk;
                *(uint4 *)(ks + key * KP + dc * 8) = ok ? kreg[i] : make_uint4(0, 0, 0, 0);
                *(uint4 *)(vs + key * att_vpitch<D>() + dc * 8) = ok ? vreg[i] : make_uint4(0, 0, 0, 0);
            }
            const int nk = next_tile(kt);  // the next tile in stream order
            if (nk >= 0) fetch(nk);
            __syncthreads();
            if (active) {
                f32x16 s;
#pragma unroll
                for (int i = 0; i < 16; ++i) s[i] = 0.0f;
#pragma unroll
                for (int kq = 0; kq < DS; ++kq) {
                    const V8 a =
                        __builtin_bit_cast(V8, *(const uint4 *)(ks + r * KP + 16 * kq + 8 * h2));
                    s = AMfma<T>::mma(a, __builtin_bit_cast(V8, qf[kq]), s);
                }
                attn_tile<T, D>(cur, s, vs, kt, q0, qrow, off, Lk, causal, scale_log2, h2, lane);
            }
        }
        if (active) {
            if (sw == 0)
                tot = cur;
            else
                attn_merge(tot, cur.m, cur.l, [&](int t, int i) { return cur.o[t][i]; });
        }
    }
    if (!qok) return;
    T *orow = out_layout ? out + ((b * Lq + qrow) * H + hq) * D
                         : out + ((b * H + hq) * Lq + qrow) * D;
    attn_store<T, D>(tot, orow, h2);
}

// The shared-K/V kernel once its grid fills half the CUs (256 CUs on MI355X);
// the split kernel below that (short prefill, decode). Same results either way.
constexpr int64_t ATT_SHARED_MIN_BLOCKS = 128;

template <typename T, int D>
int launch_attn_d(const void *q, const void *k, const void *v, void *out, int64_t B, int64_t H,
                  int64_t HK, int64_t Lq, int64_t Lk, int64_t cap, float scale_log2, int causal,
                  int out_layout, hipStream_t st) {
    const int quads = (int)ceil_div(H / HK, 4);
    const int64_t shared_blocks = B * HK * quads * ceil_div(Lq, 32);
    // causal grids pair long and short q blocks (attn_shared_kernel's zig)
    const int zig = causal && ceil_div(Lq, 32) % 2 == 0;
    if (shared_blocks >= ATT_SHARED_MIN_BLOCKS)
        attn_shared_kernel<T, D><<<(unsigned)shared_blocks, 256, 0, st>>>(
            (const T *)q, (const T *)k, (const T *)v, (T *)out, H, HK, Lq, Lk, cap, scale_log2,
            causal, out_layout, quads, zig);
    else
        attn_split_kernel<T, D><<<(unsigned)(B * H * ceil_div(Lq, 32)), 64 * ATT_STREAMS, 0, st>>>(
            (const T *)q, (const T *)k, (const T *)v, (T *)out, H, HK, Lq, Lk, cap, scale_log2,
            causal, out_layout);
    return launch_status("sdpa");
}

template <typename T>
int launch_attn(const void *q, const void *k, const void *v, void *out, int64_t B, int64_t H,
                int64_t HK, int64_t Lq, int64_t Lk, int64_t D, int64_t cap, float scale,
                int causal, int out_layout, hipStream_t st) {
    if (B * H * ceil_div(Lq, 32) == 0) return MI_OK;
    const float scale_log2 = scale * 1.4426950408889634f;
    if (D == 128)
        return launch_attn_d<T, 128>(q, k, v, out, B, H, HK, Lq, Lk, cap, scale_log2, causal,
                                     out_layout, st);
    return launch_attn_d<T, 64>(q, k, v, out, B, H, HK, Lq, Lk, cap, scale_log2, causal,
                                out_layout, st);
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int mi_sdpa(const void *q, const void *k, const void *v, void *out, int64_t B,
                       int64_t H, int64_t HK, int64_t Lq, int64_t Lk, int64_t D, int64_t kv_cap,
                       float scale, int causal, int out_layout, int dtype, void *stream) {
    if (dtype != MI_BF16 && dtype != MI_F16)
        return fail(MI_ERR_UNSUPPORTED, "sdpa covers bf16 and fp16 (dtype code %d)", dtype);
    if (D != 64 && D != 128) return fail(MI_ERR_UNSUPPORTED, "sdpa head dim %lld", (long long)D);
    if (B < 0 || H <= 0 || HK <= 0 || H % HK || Lq < 0 || Lk <= 0 || kv_cap < Lk)
        return fail(MI_ERR_ARG, "sdpa shape B=%lld H=%lld HK=%lld Lq=%lld Lk=%lld cap=%lld",
                    (long long)B, (long long)H, (long long)HK, (long long)Lq, (long long)Lk,
                    (long long)kv_cap);
    if (causal && Lq > Lk) return fail(MI_ERR_ARG, "causal sdpa needs Lq <= Lk");
    if (B * Lq && (!q || !k || !v || !out)) return fail(MI_ERR_ARG, "null pointer");
    if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(out, 8))
        return fail(MI_ERR_ARG, "q/k/v must be 16-byte aligned, out 8-byte aligned");
    hipStream_t st = as_stream(stream);
    if (dtype == MI_BF16)
        return launch_attn<bf16>(q, k, v, out, B, H, HK, Lq, Lk, D, kv_cap, scale, causal,
                                 out_layout, st);
    return launch_attn<f16>(q, k, v, out, B, H, HK, Lq, Lk, D, kv_cap, scale, causal, out_layout,
                            st);
}
