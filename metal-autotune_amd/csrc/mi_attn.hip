// Row A7: causal GQA scaled-dot-product attention (mx.fast.scaled_dot_product_attention
// with mask='causal' or none), flash-style over 32-key tiles.
//
// A workgroup is one query head (GQA: kv head of q head h is h / (H/HK),
// tests/test_graph_model_matrix.py:84-93) on one 32-query block. Its 4 waves
// split the block's key tiles: wave w takes tiles w, w + 4, w + 8, ... and
// keeps its own online-softmax state; the 4 partial states are merged at the
// end in LDS, in wave order. (A prefill of 128 tokens has 4 key tiles for its
// last block: one per wave, and 32 heads x 4 blocks = 128 workgroups.)
// Per wave and tile:
//   S^T[key][q] = K . Q^T   32x32x16 MFMA, A = K rows loaded straight into
//                           registers (16 bytes per lane and k-step), B = Q^T
//                           held in registers for the whole kernel;
//   lane (q = lane%32, half) then holds 16 of the 32 keys of its query row, so
//   the row max/sum needs one xor-32 shuffle;
//   O^T[d][q] += V^T . P^T  A = V^T from the wave's own transposed LDS tile,
//                           B = P^T straight from the S^T registers (bf16/fp16):
//                           the k order inside each MFMA is permuted to match
//                           the S^T register layout, for both operands.
// Online softmax in the log2 domain, fp32 running max/sum, one division at
// the end. Causal masking is bottom-right aligned (query i sees keys
// j <= i + Lk - Lq) and key tiles past the last visible key are skipped.
// A query row's result depends only on its global position and the keys'
// (tiles of 32 from key 0, dealt to waves by tile index), so a chunked
// prefill whose chunks start at multiples of 32 reproduces the whole prefill
// bit for bit.
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

constexpr int ATT_WAVES = 4;  // key-tile splits per workgroup

// LDS of one workgroup: the waves' V^T tiles, reused afterwards for the
// partial states of waves 1..3 (o: DT x 16 floats per lane; l, m per lane).
template <int D> struct AttnLds {
    static constexpr int KT = 32;
    static constexpr int VP = KT + 8;  // padded V^T-tile row (elements)
    static constexpr int DT = D / 32;
    static constexpr int VT_BYTES = D * VP * 2;                           // one wave's V^T tile
    static constexpr int PART_FLOATS = DT * 16 * 64 + 2 * 64;             // one wave's state
    static constexpr int BYTES = ATT_WAVES * VT_BYTES > (ATT_WAVES - 1) * PART_FLOATS * 4
                                     ? ATT_WAVES * VT_BYTES
                                     : (ATT_WAVES - 1) * PART_FLOATS * 4;
};

template <typename T, int D>
__global__ __launch_bounds__(64 * ATT_WAVES) void attn_kernel(
    const T *__restrict__ q, const T *__restrict__ k, const T *__restrict__ v,
    T *__restrict__ out, int64_t H, int64_t HK, int64_t Lq, int64_t Lk, int64_t cap,
    float scale_log2, int causal, int out_layout) {
    typedef AttnLds<D> L;
    constexpr int KT = L::KT, VP = L::VP, DT = L::DT;
    constexpr int DS = D / 16;  // MFMA k-steps over the head dim
    typedef typename Vec<T>::x8 V8;
    typedef typename Vec<T>::x4 V4;
    __shared__ __attribute__((aligned(16))) char lds[L::BYTES];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h2 = lane >> 5, r = lane & 31;
    int64_t bid = blockIdx.x;
    const int64_t nqb = ceil_div(Lq, 32);
    const int64_t qblk = bid % nqb;
    bid /= nqb;
    const int64_t hq = bid % H, b = bid / H;
    const int64_t hk = hq / (H / HK);
    const int64_t q0 = qblk * 32;
    const int64_t off = Lk - Lq;
    const int64_t qrow = q0 + r;
    const bool qok = qrow < Lq;

    uint4 qf[DS];
    {
        const T *qp = q + ((b * H + hq) * Lq + (qok ? qrow : 0)) * D + 8 * h2;
#pragma unroll
        for (int s = 0; s < DS; ++s) qf[s] = qok ? ld16(qp + 16 * s) : make_uint4(0, 0, 0, 0);
    }
    f32x16 o[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[t][i] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;

    int64_t kend = Lk;
    if (causal) {
        const int64_t last = q0 + 31 + off + 1;  // keys visible to the block's last row
        kend = last < Lk ? last : Lk;
    }
    const int ntiles = kend > 0 ? (int)ceil_div(kend, KT) : 0;
    const T *kb = k + (b * HK + hk) * cap * D;
    const T *vb = v + (b * HK + hk) * cap * D;
    T *vts = (T *)(lds + wave * L::VT_BYTES);  // this wave's V^T tile

    // A tile's loads: the K rows as MFMA A fragments (key r, head-dim chunk
    // 16 s + 8 h2), and V as 16-byte chunks (key r, chunk h2 + 2 i) for the
    // transposed LDS tile. Keys past Lk read the last key (in bounds): their
    // scores are masked and their V rows zeroed.
    constexpr int VCH = D / 16;  // V chunks per lane
    uint4 kf[DS], vreg[VCH];
    auto fetch = [&](int kt) {
        const int64_t kg = (int64_t)kt * KT + r;
        const int64_t kc = kg < Lk ? kg : Lk - 1;
#pragma unroll
        for (int s = 0; s < DS; ++s) kf[s] = ld16(kb + kc * D + 16 * s + 8 * h2);
#pragma unroll
        for (int i = 0; i < VCH; ++i) vreg[i] = ld16(vb + kc * D + (h2 + 2 * i) * 8);
    };
    if (wave < ntiles) fetch(wave);

    for (int kt = wave; kt < ntiles; kt += ATT_WAVES) {  // wave-uniform
        // V^T tile: this wave's own LDS, written and read by this wave only
        // (its LDS instructions execute in order)
        const bool vok = (int64_t)kt * KT + r < Lk;
#pragma unroll
        for (int i = 0; i < VCH; ++i) {
            const V8 vv = __builtin_bit_cast(V8, vok ? vreg[i] : make_uint4(0, 0, 0, 0));
            const int dc = h2 + 2 * i;
#pragma unroll
            for (int e = 0; e < 8; ++e) vts[(dc * 8 + e) * VP + r] = vv[e];
        }
        f32x16 s;
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = 0.0f;
#pragma unroll
        for (int st = 0; st < DS; ++st)
            s = AMfma<T>::mma(__builtin_bit_cast(V8, kf[st]), __builtin_bit_cast(V8, qf[st]), s);
        if (kt + ATT_WAVES < ntiles) fetch(kt + ATT_WAVES);  // next tile's loads under this one
        // s[i]: key kt*32 + 8*(i/4) + 4*h2 + i%4 of query row qrow. A tile
        // whose every key every row of the block sees needs no mask.
        float p[16];
        float mt = -INFINITY;
        const bool full = (int64_t)kt * KT + KT <= Lk &&
                          (!causal || (int64_t)kt * KT + KT - 1 <= q0 + off);
        const int vis_end = (int)((causal && qrow + off + 1 < Lk ? qrow + off + 1 : Lk) -
                                  (int64_t)kt * KT);  // keys [0, vis_end) of the tile
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int kl = 8 * (i / 4) + 4 * h2 + (i % 4);
            p[i] = (full || kl < vis_end) ? s[i] * scale_log2 : -INFINITY;
            mt = fmaxf(mt, p[i]);
        }
        mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
        // Lazy rescale: the exponents are taken against a running reference
        // m_run that moves only when a row's maximum passes it by more than
        // 8 (log2 units). p then stays below 2^8, where fp32 sums and the
        // bf16/fp16 P operand keep their relative precision, and the
        // accumulator rescales run only on those (wave-uniform) steps.
        const bool grow = mt > m_run + 8.0f;
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
            const float m_new = grow ? mt : m_run;
            const float corr = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
            l_run *= corr;
#pragma unroll
            for (int t = 0; t < DT; ++t)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[t][i] *= corr;
            m_run = m_new;
        }
        const bool none = m_run == -INFINITY;
        float psum = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            p[i] = none ? 0.0f : __builtin_amdgcn_exp2f(p[i] - m_run);
            psum += p[i];
        }
        l_run += psum;
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            V8 pb;
#pragma unroll
            for (int e = 0; e < 8; ++e) pb[e] = (T)p[8 * st + e];
#pragma unroll
            for (int t = 0; t < DT; ++t) {
                const T *vr = vts + (32 * t + r) * VP + 16 * st + 4 * h2;
                const V4 lo = __builtin_bit_cast(V4, *(const uint2 *)vr);
                const V4 hi = __builtin_bit_cast(V4, *(const uint2 *)(vr + 8));
                V8 a;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    a[e] = lo[e];
                    a[4 + e] = hi[e];
                }
                o[t] = AMfma<T>::mma(a, pb, o[t]);
            }
        }
    }

    // Merge: waves 1..3 leave (o, l, m) in LDS (over the V^T tiles); wave 0
    // folds them in, in wave order, each rescaled to the common maximum.
    float *part = (float *)lds;
    __syncthreads();  // every wave is done with its V^T tile
    if (wave > 0) {
        float *pp = part + (size_t)(wave - 1) * L::PART_FLOATS;
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) pp[(t * 16 + i) * 64 + lane] = o[t][i];
        pp[DT * 16 * 64 + lane] = l_run;
        pp[DT * 16 * 64 + 64 + lane] = m_run;
    }
    __syncthreads();
    if (wave > 0 || !qok) return;
    for (int w = 1; w < ATT_WAVES; ++w) {
        const float *pp = part + (size_t)(w - 1) * L::PART_FLOATS;
        const float mw = pp[DT * 16 * 64 + 64 + lane];
        if (mw == -INFINITY) continue;  // wave w saw no visible key of this row
        const float lw = pp[DT * 16 * 64 + lane];
        const float m_new = fmaxf(m_run, mw);
        const float c0 = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
        const float cw = __builtin_amdgcn_exp2f(mw - m_new);
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[t][i] = o[t][i] * c0 + pp[(t * 16 + i) * 64 + lane] * cw;
        l_run = l_run * c0 + lw * cw;
        m_run = m_new;
    }
    const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    T *orow = out_layout ? out + ((b * Lq + qrow) * H + hq) * D
                         : out + ((b * H + hq) * Lq + qrow) * D;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int blk = 0; blk < 4; ++blk) {
            float f[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) f[e] = o[t][4 * blk + e] * inv;
            st8(orow + 32 * t + 8 * blk + 4 * h2, pack4<T>(f));
        }
}

template <typename T>
int launch_attn(const void *q, const void *k, const void *v, void *out, int64_t B, int64_t H,
                int64_t HK, int64_t Lq, int64_t Lk, int64_t D, int64_t cap, float scale,
                int causal, int out_layout, hipStream_t st) {
    const int64_t blocks = B * H * ceil_div(Lq, 32);
    if (blocks == 0) return MI_OK;
    const float scale_log2 = scale * 1.4426950408889634f;
    if (D == 128)
        attn_kernel<T, 128><<<(unsigned)blocks, 64 * ATT_WAVES, 0, st>>>(
            (const T *)q, (const T *)k, (const T *)v, (T *)out, H, HK, Lq, Lk, cap, scale_log2,
            causal, out_layout);
    else
        attn_kernel<T, 64><<<(unsigned)blocks, 64 * ATT_WAVES, 0, st>>>(
            (const T *)q, (const T *)k, (const T *)v, (T *)out, H, HK, Lq, Lk, cap, scale_log2,
            causal, out_layout);
    return launch_status("sdpa");
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
