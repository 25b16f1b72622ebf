"""Region specs for the cuts the reference ships, routed to the HIP entry points.

Each builder returns a KernelSpec whose inputs are in the order the
reference's generated wrappers pass them (``_ins = [...]`` in
examples/lfm2_5_1_2b_prefill/lfm2_5_1_2b_prefill_artifact/patch/wrappers.py)
and whose outputs are the region outputs in the wrapper's order, so a
wrapper's ``_kernels.try_sized(spec, _ins)`` splice works unchanged:

  split_gate        [qmm(in_proj), split(3), mul]   wrappers.py:47-55
                    (rae66687cb9df03fe_predeq_sg2x4)   -> (C, B*x)
  residual_rmsnorm  [qmm(out_proj), add, rms_norm]  wrappers.py:67-80
                    (r95aa6c37bb25ef99_prefill_bk64)   -> (h, norm(h))
  dual              [qmm(w1), qmm(w3)]              wrappers.py:81-95
                    (r1f9367e50750eb01_unroll_hoist)   -> (gate, up)
  residual          [qmm(w2), add]                  wrappers.py:97-106
                    (r036a72bd97248ec8_s0tile_sgfullunroll) -> out

plus the single ops (qmm, dequant, rms_norm, q/k-norm + RoPE, SDPA, swiglu)
and config 1's tiny MLP as one launch (``tiny_mlp``; ``tiny_mlp_two_stage`` is the
same forward as two fp32 linear launches).

Fallback predicates state the shape contract of the entry points (packed
width and group count consistent with K, K a multiple of the group size),
the analog of the shipped specs' predicates
(``in0.shape[2] % 512 != 0 or in1.shape[1] * 8 != in0.shape[2] ...``,
kernels/*.launch.json).
"""

from __future__ import annotations

from .kernels import KernelSpec, KernelStage


def _k(i: int = 0) -> str:
    return f"in{i}.shape[in{i}.ndim - 1]"


def _quant_fallback(x: int, w: int, s: int, b: int, group_size: int, bits: int) -> str:
    per = 32 // bits
    K = _k(x)
    return (f"in{w}.ndim != 2 or in{w}.shape[1] * {per} != {K} or {K} % {group_size} != 0 "
            f"or in{s}.shape[1] * {group_size} != {K} or in{b}.shape[1] * {group_size} != {K} "
            f"or in{s}.shape[0] != in{w}.shape[0] or in{b}.shape[0] != in{w}.shape[0]")


def _lead_shape(i: int, nd: int) -> tuple[str, ...]:
    return tuple(f"in{i}.shape[{d}]" for d in range(nd - 1))


def _qparams(group_size: int, bits: int) -> tuple:
    return (("group_size", str(group_size)), ("bits", str(bits)))


def qmm(kernel_id="qmm", dtype="bfloat16", x_ndim=3, group_size=64, bits=4) -> KernelSpec:
    """[qmm]: y = x @ dequant(w)^T; inputs (x, w, scales, biases)."""
    return KernelSpec(
        kernel_id=kernel_id, name="mi_qmm_affine", input_names=("in0", "in1", "in2", "in3"),
        output_names=("out0",), source="mi_qmm_affine",
        output_shapes=((*_lead_shape(0, x_ndim), "in1.shape[0]"),), output_dtypes=(dtype,),
        template=_qparams(group_size, bits),
        fallback_predicate=f"in0.ndim != {x_ndim} or " + _quant_fallback(0, 1, 2, 3, group_size, bits))


def dequant(kernel_id="dequant", dtype="bfloat16", group_size=64, bits=4) -> KernelSpec:
    return KernelSpec(
        kernel_id=kernel_id, name="mi_affine_dequant", input_names=("in0", "in1", "in2"),
        output_names=("out0",), source="mi_affine_dequant",
        output_shapes=(("in0.shape[0]", f"in0.shape[1] * {32 // bits}"),), output_dtypes=(dtype,),
        template=_qparams(group_size, bits),
        fallback_predicate=(f"in0.ndim != 2 or (in0.shape[1] * {32 // bits}) % {group_size} != 0 "
                            f"or in1.shape[1] * {group_size} != in0.shape[1] * {32 // bits}"))


def split_gate(kernel_id="split_gate", dtype="bfloat16", group_size=64, bits=4) -> KernelSpec:
    """[qmm(in_proj), split(3), mul] -> (C, B*x); inputs (x, w, scales, biases)."""
    shape = ("in0.shape[0]", "in0.shape[1]", "in1.shape[0] / 3")
    return KernelSpec(
        kernel_id=kernel_id, name="mi_qmm_affine_split_gate",
        input_names=("in0", "in1", "in2", "in3"), output_names=("out0", "out1"),
        source="mi_qmm_affine_split_gate", output_shapes=(shape, shape),
        output_dtypes=(dtype, dtype), template=_qparams(group_size, bits),
        fallback_predicate=("in0.ndim != 3 or in1.shape[0] % 3 != 0 or "
                            + _quant_fallback(0, 1, 2, 3, group_size, bits)))


def residual_rmsnorm(kernel_id="residual_rmsnorm", dtype="bfloat16", group_size=64, bits=4,
                     eps=1e-5) -> KernelSpec:
    """[qmm(out_proj), add, rms_norm] -> (h, norm(h));
    inputs (x, w, scales, biases, residual, norm_weight)."""
    shape = ("in4.shape[0]", "in4.shape[1]", "in4.shape[2]")
    return KernelSpec(
        kernel_id=kernel_id, name="mi_qmm_affine_residual_rmsnorm",
        input_names=tuple(f"in{i}" for i in range(6)), output_names=("out0", "out1"),
        source="mi_qmm_affine_residual_rmsnorm", output_shapes=(shape, shape),
        output_dtypes=(dtype, dtype), template=(*_qparams(group_size, bits), ("eps", repr(float(eps)))),
        fallback_predicate=("in0.ndim != 3 or in4.ndim != 3 or in4.shape[2] != in1.shape[0] "
                            "or in4.shape[1] != in0.shape[1] or in4.shape[0] != in0.shape[0] "
                            "or in5.shape[0] != in1.shape[0] or "
                            + _quant_fallback(0, 1, 2, 3, group_size, bits)))


def dual(kernel_id="dual", dtype="bfloat16", group_size=64, bits=4) -> KernelSpec:
    """[qmm(w1), qmm(w3)] sharing x -> (x W1^T, x W3^T);
    inputs (x, w1, s1, b1, w3, s3, b3)."""
    return KernelSpec(
        kernel_id=kernel_id, name="mi_qmm_affine_dual",
        input_names=tuple(f"in{i}" for i in range(7)), output_names=("out0", "out1"),
        source="mi_qmm_affine_dual",
        output_shapes=(("in0.shape[0]", "in0.shape[1]", "in1.shape[0]"),
                       ("in0.shape[0]", "in0.shape[1]", "in4.shape[0]")),
        output_dtypes=(dtype, dtype), template=(*_qparams(group_size, bits), ("act", "0")),
        fallback_predicate=("in0.ndim != 3 or in4.shape[0] != in1.shape[0] "
                            "or in4.shape[1] != in1.shape[1] or "
                            + _quant_fallback(0, 1, 2, 3, group_size, bits) + " or "
                            + _quant_fallback(0, 4, 5, 6, group_size, bits)))


def dual_swiglu(kernel_id="dual_swiglu", dtype="bfloat16", group_size=64, bits=4) -> KernelSpec:
    """[qmm(gate), qmm(up), swiglu] -> silu(x W1^T) * (x W3^T) (the opaque swiglu
    call the reference leaves outside its region, fused as an epilogue)."""
    spec = dual(kernel_id, dtype, group_size, bits)
    return KernelSpec(**{**spec.__dict__, "output_names": ("out0",),
                         "output_shapes": spec.output_shapes[:1],
                         "output_dtypes": spec.output_dtypes[:1],
                         "template": (*_qparams(group_size, bits), ("act", "1"))})


def grouped3(kernel_id="grouped3", dtype="bfloat16", group_size=64, bits=4) -> KernelSpec:
    """[qmm(wq), qmm(wk), qmm(wv)] sharing x -> three outputs (the attention
    block's projections of the normed input, patch/wrappers.py:156,160,164 of
    the LFM2 artifact); inputs (x, wq, sq, bq, wk, sk, bk, wv, sv, bv). Each
    projection's N must be a multiple of 32 (else the original ops run)."""
    outs = tuple(("in0.shape[0]", "in0.shape[1]", f"in{1 + 3 * i}.shape[0]") for i in range(3))
    return KernelSpec(
        kernel_id=kernel_id, name="mi_qmm_affine_grouped3",
        input_names=tuple(f"in{i}" for i in range(10)), output_names=("out0", "out1", "out2"),
        source="mi_qmm_affine_grouped3", output_shapes=outs, output_dtypes=(dtype,) * 3,
        template=_qparams(group_size, bits),
        fallback_predicate=(
            "in0.ndim != 3 or "
            + " or ".join(f"in{1 + 3 * i}.shape[0] % 32 != 0" for i in range(3)) + " or "
            + " or ".join(_quant_fallback(0, 1 + 3 * i, 2 + 3 * i, 3 + 3 * i, group_size, bits)
                          for i in range(3))))


def residual(kernel_id="residual", dtype="bfloat16", group_size=64, bits=4) -> KernelSpec:
    """[qmm(w2), add] -> resid + x W2^T; inputs (x, w, scales, biases, residual)."""
    return KernelSpec(
        kernel_id=kernel_id, name="mi_qmm_affine_residual",
        input_names=tuple(f"in{i}" for i in range(5)), output_names=("out0",),
        source="mi_qmm_affine_residual",
        output_shapes=(("in0.shape[0]", "in0.shape[1]", "in1.shape[0]"),),
        output_dtypes=(dtype,), template=_qparams(group_size, bits),
        fallback_predicate=("in0.ndim != 3 or in4.ndim != 3 or in4.shape[2] != in1.shape[0] "
                            "or in4.shape[1] != in0.shape[1] or in4.shape[0] != in0.shape[0] or "
                            + _quant_fallback(0, 1, 2, 3, group_size, bits)))


def rms_norm(kernel_id="rms_norm", dtype="bfloat16", eps=1e-6, ndim=3) -> KernelSpec:
    shape = tuple(f"in0.shape[{d}]" for d in range(ndim))
    return KernelSpec(
        kernel_id=kernel_id, name="mi_rms_norm", input_names=("in0", "in1"),
        output_names=("out0",), source="mi_rms_norm", output_shapes=(shape,),
        output_dtypes=(dtype,), template=(("eps", repr(float(eps))),),
        fallback_predicate=f"in0.ndim != {ndim} or in1.shape[0] != {_k(0)}")


def norm_rope(kernel_id="norm_rope", dtype="bfloat16", n_heads=32, eps=1e-6, dims=128,
              base=1e6, offset=0) -> KernelSpec:
    """reshape -> rms_norm(q_norm) -> transpose -> rope: x [B, L, H*D] -> [B, H, L, D]."""
    D = f"in0.shape[2] / {n_heads}"
    return KernelSpec(
        kernel_id=kernel_id, name="mi_norm_rope", input_names=("in0", "in1"),
        output_names=("out0",), source="mi_norm_rope",
        output_shapes=(("in0.shape[0]", str(n_heads), "in0.shape[1]", D),),
        output_dtypes=(dtype,),
        template=(("n_heads", str(n_heads)), ("eps", repr(float(eps))), ("dims", str(dims)),
                  ("base", repr(float(base))), ("offset", str(offset))),
        fallback_predicate=(f"in0.ndim != 3 or in0.shape[2] % {n_heads} != 0 or "
                            f"in1.shape[0] * {n_heads} != in0.shape[2] or "
                            f"(in0.shape[2] / {n_heads}) % 2 != 0"))


def sdpa(kernel_id="sdpa", dtype="bfloat16", scale=128 ** -0.5, causal=True) -> KernelSpec:
    """mx.fast.scaled_dot_product_attention(q, k, v, scale, mask) -> [B, H, Lq, D]."""
    return KernelSpec(
        kernel_id=kernel_id, name="mi_sdpa", input_names=("in0", "in1", "in2"),
        output_names=("out0",), source="mi_sdpa",
        output_shapes=(("in0.shape[0]", "in0.shape[1]", "in0.shape[2]", "in0.shape[3]"),),
        output_dtypes=(dtype,),
        template=(("scale", repr(float(scale))), ("causal", "1" if causal else "0")),
        fallback_predicate=("in0.ndim != 4 or (in0.shape[3] != 64 and in0.shape[3] != 128) "
                            "or in0.shape[1] % in1.shape[1] != 0 or in1.shape[2] < in0.shape[2]"))


def swiglu(kernel_id="swiglu", dtype="bfloat16", ndim=3) -> KernelSpec:
    shape = tuple(f"in0.shape[{d}]" for d in range(ndim))
    return KernelSpec(kernel_id=kernel_id, name="mi_swiglu", input_names=("in0", "in1"),
                      output_names=("out0",), source="mi_swiglu", output_shapes=(shape,),
                      output_dtypes=(dtype,), fallback_predicate=f"in0.ndim != {ndim}")


def tiny_mlp(kernel_id="tiny_mlp") -> KernelSpec:
    """Config 1's whole forward as one region and one launch (fp32):
    out0 = gelu(x W1^T + b1) W2^T + b2 with inputs (x, W1, b1, W2, b2)
    (examples/tiny_mlp.py:5-6). The hidden dimension is summed in chunks
    across workgroups in a fixed order, so the region reassociates the
    two-linear stream (``reassociates``) and is checked at fp32 tolerance.
    The entry covers at most 65,535 blocks of 8 rows (M <= 524,280); larger M,
    like the other uncovered shapes, falls back to the original ops."""
    return KernelSpec(
        kernel_id=kernel_id, name="mi_gelu_mlp_f32", input_names=tuple(f"in{i}" for i in range(5)),
        output_names=("out0",), source="mi_gelu_mlp_f32",
        output_shapes=(("in0.shape[0]", "in3.shape[0]"),), output_dtypes=("float32",),
        fallback_predicate=("in0.ndim != 2 or in1.shape[1] != in0.shape[1] or "
                            "in3.shape[1] != in1.shape[0] or in0.shape[1] > 1024 or "
                            "in0.shape[1] % 4 != 0 or in1.shape[0] % 4 != 0 or "
                            "in0.shape[0] > 524280"),
        reassociates=True)


def tiny_mlp_two_stage(kernel_id="tiny_mlp_2") -> KernelSpec:
    """The same forward as a staged region of two fp32 linear launches
    (tmp0 = gelu(x W1^T + b1); out0 = tmp0 W2^T + b2), for shapes the one-launch
    region does not cover."""
    stage0 = KernelSpec(kernel_id=f"{kernel_id}_stage0", name="mi_linear_f32",
                        input_names=("in0", "in1", "in2"), output_names=("out0",),
                        source="mi_linear_f32", output_shapes=(("in0.shape[0]", "in1.shape[0]"),),
                        output_dtypes=("float32",), template=(("act", "2"),))
    stage1 = KernelSpec(kernel_id=f"{kernel_id}_stage1", name="mi_linear_f32",
                        input_names=("in0", "in1", "in2"), output_names=("out0",),
                        source="mi_linear_f32", output_shapes=(("in0.shape[0]", "in1.shape[0]"),),
                        output_dtypes=("float32",), template=(("act", "0"),))
    return KernelSpec(
        kernel_id=kernel_id, name="mi_tiny_mlp", input_names=tuple(f"in{i}" for i in range(5)),
        output_names=("out0",), source="", output_shapes=(("in0.shape[0]", "in3.shape[0]"),),
        output_dtypes=("float32",),
        fallback_predicate=("in0.ndim != 2 or in1.shape[1] != in0.shape[1] or "
                            "in3.shape[1] != in1.shape[0]"),
        stages=(KernelStage(("in0", "in1", "in2"), ("tmp0",), stage0),
                KernelStage(("tmp0", "in3", "in4"), ("out0",), stage1)),
        reassociates=True)
