/*
 * mi_qmm.h -- C ABI of the MI355X (gfx950) backend for metal-autotune's
 * quantized-matmul region path.
 *
 * The reference (shivamg05/metal-autotune) has no C ABI: its one call site is
 * autotuner_runtime/kernels.py (`call` :247-251, `try_call` :254-259,
 * `try_sized` :262-268), which hands a KernelSpec to mx.fast.metal_kernel
 * (:128-137, :212-220). Each entry below is what that call site binds for one
 * region or one library op the regions splice around; the citation names the
 * reference op or region it replaces. The Python mirror of the region API
 * (metal-autotune_amd/autotuner_runtime) binds these symbols with ctypes.
 *
 * Conventions (all entries):
 *   - Plain device pointers and element counts; no torch types.
 *   - `dtype` is the activation/scale dtype T: MI_F32, MI_F16 or MI_BF16.
 *     Packed weights are uint32 [N, K*bits/32], value j of a word at bit
 *     j*bits (LSB first); scales/biases are T [N, K/group_size].
 *   - Every array is row-contiguous unless a stride argument says otherwise.
 *   - `stream` is a hipStream_t (NULL = the null stream). Launches are
 *     stream-ordered and asynchronous; no entry synchronizes the host, and no
 *     entry allocates device memory.
 *   - Return 0 (MI_OK) or an MI_ERR_* code; mi_last_error() then holds a
 *     message for the calling thread. MI_ERR_ARG is a shape/argument the
 *     kernel does not cover (the Python side raises ValueError, as the
 *     reference's LoadedKernel.__call__ does for a fallback shape,
 *     kernels.py:196-198); MI_ERR_UNSUPPORTED is a bits/dtype/group size
 *     outside the build; MI_ERR_LAUNCH is a HIP launch error (RuntimeError,
 *     the analog of "Command buffer execution failed", ladder/child.py:44).
 */
#ifndef MI_QMM_H
#define MI_QMM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI_ABI_VERSION 6  /* 2: mi_argmax takes a workspace; 3: mi_gelu_mlp_f32;
                             4: mi_argmax_noalloc; 5: the qmm workspace entries;
                             6: mi_qmm_affine_qkv_norm_rope */

enum mi_dtype { MI_F32 = 0, MI_F16 = 1, MI_BF16 = 2 };

enum mi_status {
    MI_OK = 0,
    MI_ERR_ARG = 1,
    MI_ERR_UNSUPPORTED = 2,
    MI_ERR_LAUNCH = 3
};

enum mi_act { MI_ACT_NONE = 0, MI_ACT_SWIGLU = 1, MI_ACT_GELU = 2 };

/* ABI version of the loaded library (MI_ABI_VERSION). */
int mi_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char *mi_last_error(void);

/* mx.dequantize(w, scales, biases, group_size, bits) (affine mode):
 * out[n, k] = T(fma(s[n, k/gs], q(n, k), b[n, k/gs])), one rounding.
 * Restated at autotuner/scaffold/lower.py:1193-1211 (unpack) and the LFM2
 * artifact's predeq_sg2x4.stages/0.metal:8-14 (dequant).
 * bits in {4, 8}; group_size in {32, 64, 128}; out is T [N, K]. */
int mi_affine_dequant(const uint32_t *w, const void *scales, const void *biases, void *out,
                      int64_t N, int64_t K, int group_size, int bits, int dtype, void *stream);

/* nn.QuantizedEmbedding lookup (mlx-lm model glue, the tied embedding): rows ids[i] of
 * the quantized table dequantized into out[i, :] (T [n_ids, K]).
 * ids are int32 or int64 (`ids_are_64`); an id outside [0, N) -> MI_ERR_ARG
 * is not detectable without a sync, so out-of-range ids are clamped to N-1. */
int mi_affine_gather_dequant(const void *ids, int64_t n_ids, int ids_are_64,
                             const uint32_t *w, const void *scales, const void *biases,
                             void *out, int64_t N, int64_t K, int group_size, int bits,
                             int dtype, void *stream);

/* mx.quantized_matmul(x, w, scales, biases, transpose=True, group_size, bits,
 * mode='affine'): y[M, N] = x[M, K] @ dequant(w)^T, fp32 accumulation, one
 * rounding to T. Contract checks as scaffold/stitch.py:103-123. Small M runs a
 * wave-per-row GEMV with the factored per-group sum (the library's qmv regime,
 * stitch.py:176-230); larger M dequantizes in registers into bf16/fp16 MFMA
 * tiles (the qmm_t regime, stitch.py:233-293), each value T(fma(s, q, b)) as
 * mi_affine_dequant computes it. 4-bit tiles pre-scale s by 2^24: scales of
 * magnitude 2^104 or more (bf16 only; about 2.0e31) overflow there and give
 * inf/NaN, where mi_affine_dequant stays finite. */
int mi_qmm_affine(const void *x, const uint32_t *w, const void *scales, const void *biases,
                  void *y, int64_t M, int64_t N, int64_t K, int group_size, int bits,
                  int dtype, void *stream);

/* Region [qmm, add]: y = T(resid + T(x @ dequant(w)^T)). The LFM2 region
 * r036a72bd97248ec8_s0tile_sgfullunroll (patch/wrappers.py:97-106). */
int mi_qmm_affine_residual(const void *x, const uint32_t *w, const void *scales,
                           const void *biases, const void *resid, void *y, int64_t M,
                           int64_t N, int64_t K, int group_size, int bits, int dtype,
                           void *stream);

/* Region [qmm, add, rms_norm]: h = T(resid + T(x @ dequant(w)^T)),
 * y = rms_norm(h, norm_w, eps). Outputs (h, y): the LFM2 region
 * r95aa6c37bb25ef99_prefill_bk64 (patch/wrappers.py:67-80). N is the norm
 * width. */
int mi_qmm_affine_residual_rmsnorm(const void *x, const uint32_t *w, const void *scales,
                                   const void *biases, const void *resid,
                                   const void *norm_w, float eps, void *h, void *y,
                                   int64_t M, int64_t N, int64_t K, int group_size, int bits,
                                   int dtype, void *stream);

/* K parts. On the MFMA path (16-bit T, 8 < M <= 128, K >= 4096) the
 * accumulation over K is cut into 4 parts, each split over
 * four waves of a workgroup, and the parts are added in order -- one fixed
 * order per (M, K), whichever entry point or tile computes the output.
 * Without a workspace a workgroup runs the parts in turn. The _ws entries run
 * them as workgroups of their own, into a caller-owned fp32 workspace of
 * mi_qmm_workspace_bytes(...) bytes (16-byte aligned; contents need no
 * initialization), and a second kernel adds them and applies the region's
 * epilogue: the same results, bit for bit, on narrow-N projections (o_proj,
 * down_proj at prefill sizes) that otherwise fill a fraction of the GPU.
 * A NULL, short or misaligned workspace, or a shape with one K part, takes
 * the entry without _ws. Calls sharing a workspace must not overlap.
 * Same operations as mi_qmm_affine, mi_qmm_affine_residual and
 * mi_qmm_affine_residual_rmsnorm (kernels.py:193-220 call sites). MLX itself
 * splits K for small tile counts (qmm_splitk, whose count the reference
 * restates at scaffold/stitch.py:91-100); these parts are this library's own. */
int64_t mi_qmm_workspace_bytes(int64_t M, int64_t N, int64_t K, int group_size, int bits,
                               int dtype);  /* 0: no K parts at this shape */
int mi_qmm_affine_ws(const void *x, const uint32_t *w, const void *scales, const void *biases,
                     void *y, int64_t M, int64_t N, int64_t K, int group_size, int bits,
                     int dtype, void *workspace, int64_t workspace_bytes, void *stream);
int mi_qmm_affine_residual_ws(const void *x, const uint32_t *w, const void *scales,
                              const void *biases, const void *resid, void *y, int64_t M,
                              int64_t N, int64_t K, int group_size, int bits, int dtype,
                              void *workspace, int64_t workspace_bytes, void *stream);
int mi_qmm_affine_residual_rmsnorm_ws(const void *x, const uint32_t *w, const void *scales,
                                      const void *biases, const void *resid,
                                      const void *norm_w, float eps, void *h, void *y,
                                      int64_t M, int64_t N, int64_t K, int group_size,
                                      int bits, int dtype, void *workspace,
                                      int64_t workspace_bytes, void *stream);

/* Region [qmm, split(3), mul]: t = x @ dequant(w)^T with w of 3*D rows;
 * B, C, xs = split(t, 3, axis=-1); c_out = C, bx_out = T(B * xs)
 * (each a T [M, D]). The LFM2 region rae66687cb9df03fe_predeq_sg2x4
 * (patch/wrappers.py:47-55). N3 = 3*D. */
int mi_qmm_affine_split_gate(const void *x, const uint32_t *w, const void *scales,
                             const void *biases, void *c_out, void *bx_out, int64_t M,
                             int64_t N3, int64_t K, int group_size, int bits, int dtype,
                             void *stream);

/* Region [qmm(w1), qmm(w3)] sharing x: y1 = x @ W1^T, y2 = x @ W3^T (the LFM2
 * region r1f9367e50750eb01_unroll_hoist, patch/wrappers.py:81-95). With
 * act = MI_ACT_SWIGLU the opaque swiglu call that follows the region
 * (patch/wrappers.py:96) is applied in the epilogue instead:
 * y1 = swiglu(T(x W1^T), T(x W3^T)) and y2 is not written (may be NULL). */
int mi_qmm_affine_dual(const void *x, const uint32_t *w1, const void *s1, const void *b1,
                       const uint32_t *w2, const void *s2, const void *b2, void *y1, void *y2,
                       int64_t M, int64_t N, int64_t K, int group_size, int bits, int act,
                       int dtype, void *stream);

/* Three quantized projections of one x in one launch: y[i] = x @ dequant(w[i])^T
 * for i = 0, 1, 2, each T [M, N[i]] -- the attention block's q/k/v projections,
 * three mx.quantized_matmul calls on the same normed input
 * (examples/lfm2_5_1_2b_prefill/.../patch/wrappers.py:156,160,164), grouped
 * like the two-projection region above. Each N[i] must be a multiple of 32.
 * Results are bit-identical to three mi_qmm_affine calls. w, scales, biases,
 * y and N are arrays of 3 (host memory; the pointers they hold are device
 * pointers). */
int mi_qmm_affine_grouped3(const void *x, const uint32_t *const w[3], const void *const scales[3],
                           const void *const biases[3], void *const y[3], int64_t M,
                           const int64_t N[3], int64_t K, int group_size, int bits, int dtype,
                           void *stream);

/* mx.fast.rms_norm(x, w, eps) over the last axis of a [rows, D] array:
 * y = T(w * T(x * rsqrt(mean(x^2) + eps))). Form of
 * prefill_bk64.stages/1.metal:34-42; restated lower.py:1318-1354. */
int mi_rms_norm(const void *x, const void *w, void *y, int64_t rows, int64_t D, float eps,
                int dtype, void *stream);

/* The attention prologue (patch/wrappers.py:165-176): x viewed as
 * [B, L, H, D] with row stride x_row_stride (elements between consecutive
 * (b, l) rows); optional rms_norm over D with weight w (w == NULL skips it);
 * transpose to [B, H, L, D]; mx.fast.rope(dims=rope_dims, traditional, base,
 * scale, offset) (rope_dims == 0 skips it). Written to out laid out as
 * [B, H, out_seq_cap, D] at sequence rows [out_pos, out_pos + L): a KV cache's
 * update_and_fetch writes in place. */
int mi_norm_rope(const void *x, const void *w, void *out, int64_t B, int64_t L, int64_t H,
                 int64_t D, int64_t x_row_stride, float eps, int rope_dims, int traditional,
                 float base, float scale, int64_t offset, int64_t out_seq_cap,
                 int64_t out_pos, int dtype, void *stream);

/* The whole attention prologue in one launch (patch/wrappers.py:165-176):
 * q [B, L, Hq, D] (row stride q_row_stride) -> rms_norm(q_norm) -> rope ->
 * q_out [B, Hq, L, D]; k [B, L, Hkv, D] -> rms_norm(k_norm) -> rope -> written
 * into k_cache [B, Hkv, kv_cap, D] at rows [kv_pos, kv_pos + L); v -> copied
 * (transposed) into v_cache likewise -- the cache's update_and_fetch. Each
 * output equals the corresponding mi_norm_rope call bit for bit. */
int mi_norm_rope_qkv(const void *q, const void *k, const void *v, int64_t q_row_stride,
                     int64_t k_row_stride, int64_t v_row_stride, const void *q_norm,
                     const void *k_norm, void *q_out, void *k_cache, void *v_cache, int64_t B,
                     int64_t L, int64_t Hq, int64_t Hkv, int64_t D, float eps, int rope_dims,
                     int traditional, float base, float scale, int64_t offset, int64_t kv_cap,
                     int64_t kv_pos, int dtype, void *stream);

/* The q/k/v projections and the attention prologue in one launch
 * (patch/wrappers.py:156-176: three mx.quantized_matmul calls on the normed
 * input, then rms_norm, transpose, rope and the cache's update_and_fetch):
 * x [B * L, K] -> x @ dequant(w[i])^T for i = q, k, v (N = Hq D, Hkv D, Hkv D),
 * then exactly mi_norm_rope_qkv on those three results -- q_out [B, Hq, L, D],
 * k and v written into the caches [B, Hkv, kv_cap, D] at rows
 * [kv_pos, kv_pos + L). Every output equals mi_qmm_affine_grouped3 followed by
 * mi_norm_rope_qkv bit for bit; no intermediate q/k/v is written. Covers
 * bf16/fp16 x, 4- and 8-bit weights, D = rope_dims = 128 with 8 < B L <= 256
 * or D = rope_dims = 64 with B L >= 512 (where the fused launch is the faster;
 * the results are the same bits either way), traditional = 0, both norms,
 * K % 64 == 0
 * and 16-byte aligned norm weights and outputs; other shapes return
 * MI_ERR_UNSUPPORTED (launch nothing), and the caller runs the two entries
 * instead. w, scales and biases are arrays of 3 in host memory. */
int mi_qmm_affine_qkv_norm_rope(const void *x, const uint32_t *const w[3],
                                const void *const scales[3], const void *const biases[3],
                                const void *q_norm, const void *k_norm, void *q_out,
                                void *k_cache, void *v_cache, int64_t B, int64_t L, int64_t Hq,
                                int64_t Hkv, int64_t D, int64_t K, int group_size, int bits,
                                float eps, int rope_dims, int traditional, float base,
                                float scale, int64_t offset, int64_t kv_cap, int64_t kv_pos,
                                int dtype, void *stream);

/* mx.fast.scaled_dot_product_attention(q, k, v, scale, mask='causal'|None):
 * q [B, H, Lq, D]; k, v [B, HK, kv_cap, D] of which rows [0, Lk) are valid;
 * kv head of q head h is h / (H / HK); causal is bottom-right aligned (query
 * i sees keys j <= i + Lk - Lq). out_layout 0 writes [B, H, Lq, D], 1 writes
 * [B, Lq, H, D] (the transpose(0,2,1,3) that precedes o_proj). D in {64, 128}.
 * Region boundary: SDPA is matmul-like (regions/build.py:30-34). */
int mi_sdpa(const void *q, const void *k, const void *v, void *out, int64_t B, int64_t H,
            int64_t HK, int64_t Lq, int64_t Lk, int64_t D, int64_t kv_cap, float scale,
            int causal, int out_layout, int dtype, void *stream);

/* mlx_lm.models.activations.swiglu(g, u) = silu(g) * u, each op in T:
 * y = T(T(g * T(sigmoid(g))) * u). n elements. */
int mi_swiglu(const void *g, const void *u, void *y, int64_t n, int dtype, void *stream);

/* LFM2 short-conv core (patch/wrappers.py:56-66): pad = concat(state_in or
 * zeros [B,2,D], bx [B,L,D]); conv = depthwise conv1d(pad, w [D,3]) (kernel 3,
 * no padding, groups D); out = T(c * T(conv)); state_out = pad[:, -2:].
 * state_in and state_out may be NULL. */
int mi_shortconv(const void *bx, const void *c, const void *w, const void *state_in,
                 void *out, void *state_out, int64_t B, int64_t L, int64_t D, int dtype,
                 void *stream);

/* nn.Linear in fp32 with an optional activation (config 1's tiny MLP:
 * examples/tiny_mlp.py:5-6; mx.addmm(b, x, W^T) then nn.GELU exact erf):
 * y[M, N] = act(x[M, K] @ w[N, K]^T + bias[N]); bias may be NULL;
 * act in {MI_ACT_NONE, MI_ACT_GELU}. */
int mi_linear_f32(const float *x, const float *w, const float *bias, float *y, int64_t M,
                  int64_t N, int64_t K, int act, void *stream);

/* Config 1's whole tiny MLP as one launch (examples/tiny_mlp.py:5-6: nn.Linear ->
 * nn.GELU (exact erf) -> nn.Linear, i.e. mx.addmm(b1, x, W1^T), gelu,
 * mx.addmm(b2, h, W2^T)), fp32:
 *   y[M, N] = gelu(x[M, K] @ w1[H, K]^T + b1[H]) @ w2[N, H]^T + b2[N].
 * b1 / b2 may be NULL (zero bias). K and H multiples of 4, K <= 1024; x, w1,
 * w2 16-byte aligned. The hidden dimension is split over workgroups and the
 * last workgroup of each 8-row block adds their partial products in a fixed
 * order, so results are deterministic (a reassociation of the two-linear
 * stream, within fp32 rounding of it).
 * workspace: device memory of at least mi_gelu_mlp_f32_workspace_bytes(M, K, H, N)
 * bytes, 256-byte aligned, whose first 262,144 bytes (the per-row-block
 * counters, a fixed prefix whatever M is) are zero before its first use; every
 * call leaves them zero again, so one workspace serves calls of any M in turn.
 * M <= 524,280 (65,535 row blocks). Calls that share a workspace must not
 * overlap. */
int64_t mi_gelu_mlp_f32_workspace_bytes(int64_t M, int64_t K, int64_t H, int64_t N);
int mi_gelu_mlp_f32(const float *x, const float *w1, const float *b1, const float *w2,
                    const float *b2, float *y, int64_t M, int64_t K, int64_t H, int64_t N,
                    void *workspace, int64_t workspace_bytes, void *stream);

/* Greedy sampling (mlx-lm glue; mx.argmax(logits, axis=-1) in mlx-lm's
 * generate loop): out[r] = argmax over x[r, 0:V]; the lowest index wins a
 * tie; NaN never wins; a row with no non-NaN value gives 0. out is int32
 * [rows]; V < 2^31.
 * workspace: device memory of at least mi_argmax_workspace_bytes(rows, V)
 * bytes, 8-byte aligned, rows <= 65535; with it each row is split over many
 * workgroups (two launches). NULL: one workgroup per row (one launch). Same
 * result either way. Calls that share a workspace must not overlap. */
int64_t mi_argmax_workspace_bytes(int64_t rows, int64_t V);
int mi_argmax(const void *x, int32_t *out, int64_t rows, int64_t V, int dtype, void *workspace,
              int64_t workspace_bytes, void *stream);

/* No counterpart in the reference. mi_argmax for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc): no workspace argument and no allocation. The
 * per-span partials live in a fixed device array of the library, 8192
 * entries (64 KiB) per GPU, looked up on the first call on a device and held
 * until the process ends. rows x spans must fit it (spans = ceil(V * size /
 * 8192 bytes) for 16-byte-aligned rows, e.g. at most 215 rows of
 * V = 151936 bf16), else MI_ERR_ARG. Same result as mi_argmax. Calls that
 * overlap on one GPU race on that array. */
int mi_argmax_noalloc(const void *x, int32_t *out, int64_t rows, int64_t V, int dtype,
                      void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MI_QMM_H */
