/*
 * CPU oracle for the affine quantized-matmul path -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library, and only as the checker (or the timed CPU baseline). The
 * product path (the HIP library) never calls it.
 *
 * What it restates (file:line into the reference, shivamg05/metal-autotune):
 *
 *   orc_dequant_f32   affine unpack + dequant. Unpack order from
 *                     autotuner/scaffold/lower.py:1193-1211 (value j of a word
 *                     is (p >> (j*bits)) & mask, k = word*(32/bits) + j,
 *                     group = k / group_size). Dequant form fma(s, q, b) in
 *                     fp32 from examples/lfm2_5_1_2b_prefill/
 *                     lfm2_5_1_2b_prefill_artifact/kernels/
 *                     rae66687cb9df03fe_predeq_sg2x4.stages/0.metal:8-14 and
 *                     r036a72bd97248ec8_s0tile_sgfullunroll.stages/0.metal:19-25
 *                     (kernels that passed the reference's bitwise whole-model
 *                     check). The single rounding to the activation dtype is
 *                     done by the caller (oracle/__init__.py), the same
 *                     float -> T conversion the kernels perform.
 *
 *   orc_qmm_factored  quantized matmul in the per-group factored form
 *                     acc += s * sum(x*q) + b * sum(x), fp32, sequential in k
 *                     within a group, groups in order: lower.py:1179-1233
 *                     (_emit_qmm). Returns fp32; the caller rounds to T.
 *
 * Built by oracle/Makefile with -ffp-contract=off so a*b+c is never fused
 * behind the restatement's back; fmaf is called explicitly where the
 * reference fuses.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint32_t q_at(const uint32_t *row, int64_t k, int bits) {
    const int per = 32 / bits;
    const uint32_t mask = (bits == 32) ? 0xffffffffu : ((1u << bits) - 1u);
    return (row[k / per] >> ((k % per) * bits)) & mask;
}

int orc_abi_version(void) { return 1; }

/* out[n*K + k] = fmaf(s[n, k/gs], q(n,k), b[n, k/gs]) in fp32. */
void orc_dequant_f32(const uint32_t *w, const float *s, const float *b, float *out,
                     int64_t N, int64_t K, int gs, int bits) {
    const int64_t wpr = K * bits / 32;
    const int64_t G = K / gs;
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
        const uint32_t *row = w + n * wpr;
        for (int64_t k = 0; k < K; ++k) {
            const float q = (float)q_at(row, k, bits);
            out[n * K + k] = fmaf(s[n * G + k / gs], q, b[n * G + k / gs]);
        }
    }
}

/*
 * y[m*N + n] = sum_g ( s[n,g] * sum_{k in g} x[m,k]*q(n,k) + b[n,g] * sum_{k in g} x[m,k] )
 * x holds the activation values (already representable in T) as fp32.
 * nthreads <= 0 keeps the OpenMP default.
 */
void orc_qmm_factored(const float *x, const uint32_t *w, const float *s, const float *b,
                      float *y, int64_t M, int64_t N, int64_t K, int gs, int bits,
                      int nthreads) {
    const int64_t wpr = K * bits / 32;
    const int64_t G = K / gs;
    /* xt[k*M + m]: the inner loop runs over m so independent rows vectorize
     * while each (m, n, g) sum stays sequential in k. */
    float *xt = (float *)malloc(sizeof(float) * (size_t)(K * M));
    float *xs = (float *)malloc(sizeof(float) * (size_t)(G * M)); /* sum(x) per group */
    for (int64_t m = 0; m < M; ++m)
        for (int64_t k = 0; k < K; ++k) xt[k * M + m] = x[m * K + k];
    for (int64_t g = 0; g < G; ++g)
        for (int64_t m = 0; m < M; ++m) {
            float dx = 0.0f;
            for (int64_t k = g * gs; k < (g + 1) * gs; ++k) dx += x[m * K + k];
            xs[g * M + m] = dx;
        }
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#endif
#pragma omp parallel
    {
        float *acc = (float *)malloc(sizeof(float) * (size_t)M);
        float *dq = (float *)malloc(sizeof(float) * (size_t)M);
        float *qf = (float *)malloc(sizeof(float) * (size_t)gs);
#pragma omp for schedule(static)
        for (int64_t n = 0; n < N; ++n) {
            const uint32_t *row = w + n * wpr;
            for (int64_t m = 0; m < M; ++m) acc[m] = 0.0f;
            for (int64_t g = 0; g < G; ++g) {
                for (int64_t j = 0; j < gs; ++j) qf[j] = (float)q_at(row, g * gs + j, bits);
                for (int64_t m = 0; m < M; ++m) dq[m] = 0.0f;
                for (int64_t j = 0; j < gs; ++j) {
                    const float qv = qf[j];
                    const float *xr = xt + (g * gs + j) * M;
                    for (int64_t m = 0; m < M; ++m) dq[m] += xr[m] * qv;
                }
                const float sc = s[n * G + g], bi = b[n * G + g];
                const float *dx = xs + g * M;
                for (int64_t m = 0; m < M; ++m) acc[m] += sc * dq[m] + bi * dx[m];
            }
            for (int64_t m = 0; m < M; ++m) y[m * N + n] = acc[m];
        }
        free(acc);
        free(dq);
        free(qf);
    }
    free(xt);
    free(xs);
}
