// Row A7: causal GQA scaled-dot-product attention (mx.fast.scaled_dot_product_attention
// with mask='causal' or none), flash-style with 32-key tiles staged in LDS.
//
// A workgroup is 4 waves = 4 query heads that share one kv head (GQA: kv head
// of q head h is h / (H/HK), tests/test_graph_model_matrix.py:84-93), all on
// the same 32-query block, so each K/V tile is read from HBM once per group.
// Per wave and tile:
//   S^T[key][q] = K . Q^T   32x32x16 MFMA, A = K rows from LDS, B = Q^T held
//                           in registers for the whole kernel;
//   lane (q = lane%32, half) then holds 16 of the 32 keys of its query row, so
//   the row max/sum needs one xor-32 shuffle;
//   O^T[d][q] += V^T . P^T  A = V^T from a transposed LDS tile, B = P^T
//                           straight from the S^T registers (bf16/fp16): the
//                           k order inside each MFMA is permuted to match the
//                           S^T register layout, for both operands.
// Online softmax in the log2 domain, fp32 running max/sum, one division at
// the end. Causal masking is bottom-right aligned (query i sees keys
// j <= i + Lk - Lq) and key tiles past the last visible key are skipped.
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

template <typename T, int D>
__global__ __launch_bounds__(256) void attn_kernel(const T *__restrict__ q,
                                                   const T *__restrict__ k,
                                                   const T *__restrict__ v, T *__restrict__ out,
                                                   int64_t H, int64_t HK, int64_t Lq, int64_t Lk,
                                                   int64_t cap, float scale_log2, int causal,
                                                   int out_layout, int quads) {
    constexpr int KT = 32;      // keys per tile
    constexpr int KP = D + 8;   // padded K-tile row (elements)
    constexpr int VP = KT + 8;  // padded V^T-tile row (elements)
    constexpr int DS = D / 16;  // MFMA k-steps over the head dim
    constexpr int DT = D / 32;  // 32-wide output tiles over the head dim
    typedef typename Vec<T>::x8 V8;
    typedef typename Vec<T>::x4 V4;
    __shared__ __attribute__((aligned(16))) T ks[KT * KP];
    __shared__ __attribute__((aligned(16))) T vts[D * VP];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h2 = lane >> 5, r = lane & 31;
    int64_t bid = blockIdx.x;
    const int64_t nqb = ceil_div(Lq, 32);
    const int64_t qblk = bid % nqb;
    bid /= nqb;
    const int quad = (int)(bid % quads);
    bid /= quads;
    const int64_t hk = bid % HK, b = bid / HK;
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

    // K/V tile staging: each thread owns CH 16-byte chunks of a tile. The
    // chunks of tile kt + 1 are loaded into registers while tile kt computes,
    // so a tile's global-load latency overlaps the previous tile's MFMAs.
    // Consecutive lanes take consecutive keys: the transposed V stores of a
    // wave then hit consecutive 2-byte LDS addresses (with the head-dim chunk
    // fastest, 16 lanes would store into one bank).
    constexpr int CH = KT * D / 8 / 256;
    uint4 kreg[CH], vreg[CH];
    auto fetch = [&](int kt) {
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int c = threadIdx.x + 256 * i;
            const int key = c % KT, dc = c / KT;
            const int64_t kg = (int64_t)kt * KT + key;
            const int64_t kc = kg < Lk ? kg : Lk - 1;  // in bounds; masked below
            kreg[i] = ld16(kb + kc * D + dc * 8);
            vreg[i] = ld16(vb + kc * D + dc * 8);
        }
    };
    if (ntiles > 0) fetch(0);

    for (int kt = 0; kt < ntiles; ++kt) {
        __syncthreads();  // every wave is done with tile kt - 1
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int c = threadIdx.x + 256 * i;
            const int key = c % KT, dc = c / KT;
            const bool ok = (int64_t)kt * KT + key < Lk;
            *(uint4 *)(ks + key * KP + dc * 8) = ok ? kreg[i] : make_uint4(0, 0, 0, 0);
            const V8 vv = __builtin_bit_cast(V8, ok ? vreg[i] : make_uint4(0, 0, 0, 0));
#pragma unroll
            for (int e = 0; e < 8; ++e) vts[(dc * 8 + e) * VP + key] = vv[e];
        }
        if (kt + 1 < ntiles) fetch(kt + 1);  // workgroup-uniform
        __syncthreads();
        if (!active) continue;

        f32x16 s;
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = 0.0f;
#pragma unroll
        for (int st = 0; st < DS; ++st) {
            const V8 a = __builtin_bit_cast(V8, *(const uint4 *)(ks + r * KP + 16 * st + 8 * h2));
            s = AMfma<T>::mma(a, __builtin_bit_cast(V8, qf[st]), s);
        }
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
        // bf16/fp16 P operand keep their relative precision, and the 64
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
    if (!qok) return;
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
    const int64_t rep = H / HK;
    const int quads = (int)ceil_div(rep, 4);
    const int64_t blocks = B * HK * quads * ceil_div(Lq, 32);
    if (blocks == 0) return MI_OK;
    const float scale_log2 = scale * 1.4426950408889634f;
    if (D == 128)
        attn_kernel<T, 128><<<(unsigned)blocks, 256, 0, st>>>((const T *)q, (const T *)k,
                                                              (const T *)v, (T *)out, H, HK, Lq,
                                                              Lk, cap, scale_log2, causal,
                                                              out_layout, quads);
    else
        attn_kernel<T, 64><<<(unsigned)blocks, 256, 0, st>>>((const T *)q, (const T *)k,
                                                             (const T *)v, (T *)out, H, HK, Lq,
                                                             Lk, cap, scale_log2, causal,
                                                             out_layout, quads);
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
