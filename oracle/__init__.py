"""CPU oracle for the quantized-matmul region path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (or as the timed CPU
baseline). The product path -- the HIP library behind ``autotuner_runtime`` --
never imports or calls anything here, and fails loudly when its extension is
missing instead of falling back to this code.

The reference (shivamg05/metal-autotune) reaches this arithmetic through the
un-vendored ``mlx==0.32.2`` wheel (``uv.lock:575-577``) and ``mlx-lm==0.31.3``
model glue (``uv.lock:611-612``). Neither is installed here, so each function
restates the semantics the reference's own files fix, citing them, and is pinned
by the checks listed per function (tests/test_oracle.py holds them).

Values of a low-precision dtype T are carried as float32 numpy arrays whose
entries are exactly representable in T; ``round_to`` performs the one
round-to-nearest-even conversion a kernel's ``T(float)`` cast performs.

Pins (all in tests/test_oracle.py):
  dequantize          C fmaf path == independent numpy path (bf16/fp16 scales,
                      where s*q is exact in fp32); closed forms q in
                      [0, 2^bits-1], LSB-first nibble order against a
                      hand-packed word, s=0 -> b exactly, one-hot rows.
  quantized_matmul    brute-force float64 x @ W^T vs the C factored restatement
                      (lower.py:1179-1233); x = 0 -> 0 exactly; s = 0 ->
                      per-group sum(x)*b closed form; one-hot x -> dequantized
                      row exactly.
  rms_norm            eps-placement KAT of tests/test_scaffold.py:205-220
                      (eps 0.25, weight 1.5, closed form); constant row ->
                      w / sqrt(1 + eps/c^2) closed form.
  rope                offset 0 / position 0 is the identity; per-pair norm is
                      preserved; dims beyond `dims` pass through; a 90-degree
                      rotation case checked against the textbook matrix;
                      traditional vs non-traditional agree after the pair
                      permutation.
  sdpa                row 0 of a causal prefill returns v[key 0]; uniform
                      scores give the running mean of v; GQA head mapping
                      h // (H/HK) against per-head repeat; equals a brute
                      force double loop on a tiny case.
  swiglu, gelu        closed forms (math.erf) on scalars; GELU known values
                      (Phi(1) = 0.8413447460685429).
  tiny_mlp            one-hot W1/W2 closed form with nonzero b1 and b2
                      (y = c * gelu(x[k] + b1[j]) + b2, GELU by math.erf per
                      scalar); zero W2 -> b2 exactly.
  norm_rope (layout)  head h of the output == rms_norm then rope of the
                      contiguous input slice [h*D, (h+1)*D) with positions
                      along L; permuting input heads permutes output heads.
  shortconv           direct 3-tap sum against a hand-computed case; state
                      carries the last two rows; chunked == whole sequence.
  qwen3_layer         op order of mlx-lm's qwen3 decoder (un-vendored; the
                      reference's tests/fixtures/llama_ish.py:25-39 states the
                      same residual structure); pinned by structure checks:
                      zero o_proj/down_proj -> identity exactly; decode at
                      offset L against a cache filled by the prefix == the
                      last row of an (L+1)-token prefill, and a wrong offset
                      fails that bar. Bitwise agreement with MLX's own layer
                      (its fused-kernel rounding) is parity unpinned.
  qwen3_forward       no-layer case: tied head over the dequantized table
                      row of the last id.
  lfm2_conv_layer,    op streams of the reference's LFM2 wrappers (cited per
  lfm2_attn_layer     function), composed of the pinned primitives above;
                      pinned by structure checks: zero out_proj and w2 ->
                      identity exactly; a conv layer run in two chunks with
                      the state carried == one run over the whole sequence;
                      an attention decode at offset L == the last row of an
                      (L+1)-token prefill. Bitwise agreement with MLX's own
                      LFM2 layers is parity unpinned.
"""

from __future__ import annotations

import ctypes
import math
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB = None

FLOAT_DTYPES = ("float32", "float16", "bfloat16")


# ----------------------------------------------------------------------------
# dtype helpers


def _bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round to nearest even; NaN stays NaN."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32)
    nan = np.isnan(x)
    if nan.any():
        rounded = np.where(nan, ((u >> 16) | 0x40).astype(np.uint32), rounded)
    return (rounded & 0xFFFF).astype(np.uint16)


def bf16_from_bits(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_to(x, dtype: str) -> np.ndarray:
    """One float -> T conversion (RNE), returned as float32 values of T."""
    x = np.asarray(x)
    if dtype == "float32":
        return x.astype(np.float32)
    x32 = x.astype(np.float32)
    if dtype == "float16":
        return x32.astype(np.float16).astype(np.float32)
    if dtype == "bfloat16":
        return bf16_from_bits(_bf16_bits(x32))
    raise ValueError(f"unsupported dtype {dtype!r}")


# ----------------------------------------------------------------------------
# C library (oracle/oracle.c)


def lib():
    """The compiled C restatement; built by `make -C oracle` (build() runs it)."""
    global _LIB
    if _LIB is None:
        path = _HERE / "liboracle.so"
        if not path.exists():
            raise RuntimeError(f"{path} is missing: run `make -C {_HERE}` first")
        L = ctypes.CDLL(str(path))
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        C = ctypes.c_int
        L.orc_dequant_f32.argtypes = [P, P, P, P, I64, I64, C, C]
        L.orc_dequant_f32.restype = None
        L.orc_qmm_factored.argtypes = [P, P, P, P, P, I64, I64, I64, C, C, C]
        L.orc_qmm_factored.restype = None
        _LIB = L
    return _LIB


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


# ----------------------------------------------------------------------------
# A1: affine packing, quantizer (the build's rule), dequant


def pack(q: np.ndarray, bits: int) -> np.ndarray:
    """q[N, K] integer codes -> uint32[N, K*bits/32], value j of a word at bit
    j*bits (LSB first): the layout lower.py:1193-1211 unpacks."""
    q = np.asarray(q, dtype=np.uint64)
    N, K = q.shape
    per = 32 // bits
    if K % per:
        raise ValueError(f"K={K} does not pack at {bits} bits")
    q = q.reshape(N, K // per, per)
    shifts = (np.arange(per, dtype=np.uint64) * bits)[None, None, :]
    return (q << shifts).sum(axis=-1).astype(np.uint32)


def unpack(wq: np.ndarray, bits: int) -> np.ndarray:
    """uint32[N, W] -> uint8/uint16 codes [N, W*32/bits] (lower.py:1199-1211)."""
    wq = np.asarray(wq, dtype=np.uint32)
    N, W = wq.shape
    per = 32 // bits
    mask = np.uint32((1 << bits) - 1)
    shifts = (np.arange(per, dtype=np.uint32) * bits)[None, None, :]
    q = (wq[:, :, None] >> shifts) & mask
    return q.reshape(N, W * per).astype(np.uint16)


def quantize_affine(w: np.ndarray, group_size: int = 64, bits: int = 4,
                    dtype: str = "bfloat16"):
    """The build's affine quantizer (NOT mx.quantize, whose exact scale/bias
    choice only an MLX import could pin): per group of `group_size` values
    along K, s = (max - min) / (2^bits - 1), b = min, both rounded to T;
    q = clip(round((w - b) / s)). Its outputs are the path's INPUTS (packed w,
    scales, biases), so the rule does not enter any parity claim.

    Returns (wq uint32[N, K*bits/32], scales f32[N, K/gs], biases f32[N, K/gs])
    with scales/biases holding values of T."""
    w = np.asarray(w, dtype=np.float32)
    N, K = w.shape
    if K % group_size:
        raise ValueError("K must be a multiple of group_size")
    levels = (1 << bits) - 1
    g = w.reshape(N, K // group_size, group_size)
    lo = g.min(axis=-1)
    hi = g.max(axis=-1)
    s = round_to((hi - lo) / np.float32(levels), dtype)
    b = round_to(lo, dtype)
    safe = np.where(s == 0, np.float32(1), s)
    q = np.rint((g - b[..., None]) / safe[..., None])
    q = np.clip(q, 0, levels).astype(np.uint32).reshape(N, K)
    return pack(q, bits), s.astype(np.float32), b.astype(np.float32)


def dequantize(wq, scales, biases, group_size: int, bits: int, dtype: str) -> np.ndarray:
    """A1: W[n, k] = T(fma(s, q, b)) -- one fp32 fma, one rounding to T
    (predeq_sg2x4.stages/0.metal:13-14, s0tile_sgfullunroll.stages/0.metal:21-25).
    Computed by the C library with an explicit fmaf."""
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    s = np.ascontiguousarray(scales, dtype=np.float32)
    b = np.ascontiguousarray(biases, dtype=np.float32)
    N = wq.shape[0]
    K = wq.shape[1] * 32 // bits
    out = np.empty((N, K), dtype=np.float32)
    lib().orc_dequant_f32(_ptr(wq), _ptr(s), _ptr(b), _ptr(out), N, K, group_size, bits)
    return round_to(out, dtype)


def dequantize_numpy(wq, scales, biases, group_size: int, bits: int, dtype: str) -> np.ndarray:
    """Independent restatement of `dequantize` for bf16/fp16 scales: s*q is
    exact in fp32 there (<= 11 + 4 significant bits), so the fp32 sum s*q + b
    rounds exactly as fmaf does. Used to pin the C path."""
    if dtype == "float32":
        raise ValueError("fp32 scales need a true fma; use dequantize()")
    q = unpack(wq, bits).astype(np.float32)
    N, K = q.shape
    s = np.repeat(np.asarray(scales, np.float32), group_size, axis=1)
    b = np.repeat(np.asarray(biases, np.float32), group_size, axis=1)
    return round_to(s * q + b, dtype)


# ----------------------------------------------------------------------------
# A2-A4: quantized matmul


def quantized_matmul(x, wq, scales, biases, group_size: int, bits: int, dtype: str,
                     *, dequant_first: bool = True) -> np.ndarray:
    """y = x @ W^T with W the dequantized weights, float64 accumulation, one
    rounding to T. dequant_first=True rounds W to T before the product (MLX's
    qmm_t regime: dequantize into T tiles, then MMA; stitch.py:233-293);
    False keeps s*q+b unrounded (the qmv regime's factored sum,
    stitch.py:176-230)."""
    x = np.asarray(x, dtype=np.float32)
    if dequant_first:
        W = dequantize(wq, scales, biases, group_size, bits, dtype).astype(np.float64)
    else:
        q = unpack(wq, bits).astype(np.float64)
        s = np.repeat(np.asarray(scales, np.float64), group_size, axis=1)
        b = np.repeat(np.asarray(biases, np.float64), group_size, axis=1)
        W = s * q + b
    lead = x.shape[:-1]
    y = x.reshape(-1, x.shape[-1]).astype(np.float64) @ W.T
    return round_to(y, dtype).reshape(*lead, W.shape[0])


def qmm_factored(x, wq, scales, biases, group_size: int, bits: int, dtype: str,
                 nthreads: int = 0) -> np.ndarray:
    """The reference's restated algorithm (lower.py:1179-1233): fp32, per-group
    acc += s*sum(x*q) + b*sum(x), rounded to T. C implementation."""
    x = np.asarray(x, dtype=np.float32)
    lead = x.shape[:-1]
    x2 = np.ascontiguousarray(x.reshape(-1, x.shape[-1]))
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    s = np.ascontiguousarray(scales, dtype=np.float32)
    b = np.ascontiguousarray(biases, dtype=np.float32)
    M, K = x2.shape
    N = wq.shape[0]
    y = np.empty((M, N), dtype=np.float32)
    lib().orc_qmm_factored(_ptr(x2), _ptr(wq), _ptr(s), _ptr(b), _ptr(y), M, N, K,
                           group_size, bits, nthreads)
    return round_to(y, dtype).reshape(*lead, N)


# ----------------------------------------------------------------------------
# A5: RMSNorm


def rms_norm(x, w, eps: float, dtype: str) -> np.ndarray:
    """mx.fast.rms_norm over the last axis: inv = rsqrt(mean(x^2) + eps),
    y = T(w * T(x * inv)) -- two roundings, the form of
    r95aa6c37bb25ef99_prefill_bk64.stages/1.metal:34-42 (passed `exact`) and
    lower.py:1318-1354. Sums in float64."""
    x64 = np.asarray(x, dtype=np.float64)
    inv = 1.0 / np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True) + eps)
    xn = round_to(x64 * inv, dtype).astype(np.float64)
    return round_to(np.asarray(w, np.float64) * xn, dtype)


# ----------------------------------------------------------------------------
# A6: RoPE and the q/k-norm + RoPE region


def rope(x, dims: int, traditional: bool, base: float, scale: float, offset: int,
         dtype: str) -> np.ndarray:
    """mx.fast.rope on [..., L, D]: position = (l + offset) * scale along axis
    -2, theta_j = position * base^(-2j/dims); non-traditional pairs (j, j+dims/2),
    traditional pairs (2j, 2j+1); tail beyond `dims` copies through
    (lower.py:515-544, 1236-1293). Float64 angles."""
    x64 = np.asarray(x, dtype=np.float64)
    L, D = x64.shape[-2], x64.shape[-1]
    half = dims // 2
    pos = (np.arange(L, dtype=np.float64) + offset) * scale
    inv = base ** (-(2.0 * np.arange(half, dtype=np.float64)) / dims)
    th = pos[:, None] * inv[None, :]
    c, s = np.cos(th), np.sin(th)
    out = x64.copy()
    if traditional:
        a, b = x64[..., 0:dims:2], x64[..., 1:dims:2]
        out[..., 0:dims:2] = a * c - b * s
        out[..., 1:dims:2] = a * s + b * c
    else:
        a, b = x64[..., :half], x64[..., half:dims]
        out[..., :half] = a * c - b * s
        out[..., half:dims] = a * s + b * c
    return round_to(out, dtype)


def norm_rope(x, w, eps: float, n_heads: int, dims: int, base: float, offset: int,
              dtype: str, traditional: bool = False, scale: float = 1.0) -> np.ndarray:
    """The Qwen3 / LFM2 attention prologue (patch/wrappers.py:165-176):
    reshape [B, L, H*D] -> [B, L, H, D], rms_norm over D (skipped when w is
    None), transpose to [B, H, L, D], rope. Returns [B, H, L, D]."""
    x = np.asarray(x, dtype=np.float32)
    B, L, HD = x.shape
    D = HD // n_heads
    t = x.reshape(B, L, n_heads, D)
    if w is not None:
        t = rms_norm(t, w, eps, dtype)
    t = np.transpose(t, (0, 2, 1, 3))
    if dims:
        t = rope(t, dims, traditional, base, scale, offset, dtype)
    return np.ascontiguousarray(t)


# ----------------------------------------------------------------------------
# A7: causal GQA attention


def sdpa(q, k, v, scale: float, causal: bool, dtype: str) -> np.ndarray:
    """mx.fast.scaled_dot_product_attention with mask='causal' (or none):
    q [B, H, Lq, D], k/v [B, HK, Lk, D]; kv head of q head h is h // (H/HK)
    (tests/test_graph_model_matrix.py:84-93); causal is bottom-right aligned,
    query i sees keys j <= i + (Lk - Lq); stable softmax (max, exp, sum,
    divide: lower.py:1453-1490) in float64, one rounding to T."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, H, Lq, D = q.shape
    HK, Lk = k.shape[1], k.shape[2]
    rep = H // HK
    out = np.empty((B, H, Lq, v.shape[-1]), dtype=np.float64)
    if causal:
        qi = np.arange(Lq)[:, None] + (Lk - Lq)
        mask = np.arange(Lk)[None, :] <= qi
    for b in range(B):
        for h in range(H):
            kv = h // rep
            s = (q[b, h] @ k[b, kv].T) * scale
            if causal:
                s = np.where(mask, s, -np.inf)
            m = s.max(axis=-1, keepdims=True)
            p = np.exp(s - m)
            out[b, h] = (p @ v[b, kv]) / p.sum(axis=-1, keepdims=True)
    return round_to(out, dtype)


# ----------------------------------------------------------------------------
# A8 / A10: activations


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def swiglu(g, u, dtype: str) -> np.ndarray:
    """mlx_lm.models.activations.swiglu = silu(gate) * up, silu(g) = g*sigmoid(g),
    each MLX op returning T: T(T(g * T(sigmoid(g))) * u). Float64 inside."""
    g64 = np.asarray(g, np.float64)
    sig = round_to(_sigmoid(g64), dtype).astype(np.float64)
    act = round_to(g64 * sig, dtype).astype(np.float64)
    return round_to(act * np.asarray(u, np.float64), dtype)


def gelu(x) -> np.ndarray:
    """nn.GELU (approx='none'): x * (1 + erf(x / sqrt(2))) / 2, float64."""
    x64 = np.asarray(x, np.float64)
    erf = np.vectorize(math.erf)
    return x64 * (1.0 + erf(x64 / math.sqrt(2.0))) / 2.0


def tiny_mlp(x, w1, b1, w2, b2) -> np.ndarray:
    """Config 1 / row A10: Linear -> GELU -> Linear in fp32 semantics
    (examples/tiny_mlp.py:5-6); float64 inside, one fp32 rounding at the end."""
    x64 = np.asarray(x, np.float64)
    h = x64 @ np.asarray(w1, np.float64).T + np.asarray(b1, np.float64)
    y = gelu(h) @ np.asarray(w2, np.float64).T + np.asarray(b2, np.float64)
    return y.astype(np.float32)


# ----------------------------------------------------------------------------
# A9: LFM2 gated short-conv


def split_gate(y3, dtype: str):
    """[qmm(in_proj), split(3), mul] outputs (patch/wrappers.py:47-55):
    B, C, x = split(y, 3, axis=-1); returns (C, T(B*x))."""
    y3 = np.asarray(y3, np.float32)
    D = y3.shape[-1] // 3
    Bm, Cm, xm = y3[..., :D], y3[..., D:2 * D], y3[..., 2 * D:]
    return Cm.copy(), round_to(Bm.astype(np.float64) * xm.astype(np.float64), dtype)


def shortconv(bx, c, w, state, dtype: str):
    """concatenate([state or zeros(B,2,D), Bx]) -> depthwise conv1d, kernel 3,
    no padding, groups D -> C * conv (patch/wrappers.py:56-66).
    bx, c [B, L, D]; w [D, 3] (MLX conv1d weight [D, 3, 1] squeezed);
    state [B, 2, D] or None. Returns (out [B, L, D], new_state [B, 2, D])."""
    bx = np.asarray(bx, np.float64)
    B, L, D = bx.shape
    st = np.zeros((B, 2, D)) if state is None else np.asarray(state, np.float64)
    pad = np.concatenate([st, bx], axis=1)
    w = np.asarray(w, np.float64)
    conv = pad[:, 0:L] * w[:, 0] + pad[:, 1:L + 1] * w[:, 1] + pad[:, 2:L + 2] * w[:, 2]
    conv = round_to(conv, dtype).astype(np.float64)
    out = round_to(np.asarray(c, np.float64) * conv, dtype)
    return out, round_to(pad[:, -2:], dtype)


# ----------------------------------------------------------------------------
# A12: model composition (mlx-lm qwen3 op order, every op's output in T)


def _qmm_auto(x, lin, gs, bits, dtype):
    """MLX routes small M to the factored qmv and larger M to dequantize-then-
    matmul (stitch.py:74-100); the oracle follows the same split."""
    wq, s, b = lin
    M = int(np.prod(x.shape[:-1]))
    if M <= 8:
        return qmm_factored(x, wq, s, b, gs, bits, dtype)
    return quantized_matmul(x, wq, s, b, gs, bits, dtype)


def qwen3_layer(x, W: dict, cfg, offset: int, kcache, vcache, dtype: str = "bfloat16",
                qmm=None):
    """One Qwen3 decoder layer (mlx-lm qwen3.py order): h = x + attn(norm(x)),
    out = h + mlp(norm(h)). W holds (wq, scales, biases) per projection and norm
    weights; kcache/vcache [1, HK, cap, D] float32 are written at
    [offset, offset + L). Returns the layer output [1, L, hidden].
    qmm(x, lin) -> projection replaces the default routing (_qmm_auto); the
    CPU baseline passes the C factored restatement for every projection."""
    gs, bits, eps = cfg.group_size, cfg.bits, cfg.rms_norm_eps
    proj = qmm or (lambda a, lin: _qmm_auto(a, lin, gs, bits, dtype))
    H, HK, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    L = x.shape[1]
    xn = rms_norm(x, W["input_layernorm"], eps, dtype)
    q = proj(xn, W["q_proj"])
    k = proj(xn, W["k_proj"])
    v = proj(xn, W["v_proj"])
    qr = norm_rope(q, W["q_norm"], eps, H, D, cfg.rope_theta, offset, dtype)
    kcache[:, :, offset:offset + L] = norm_rope(k, W["k_norm"], eps, HK, D, cfg.rope_theta,
                                                offset, dtype)
    vcache[:, :, offset:offset + L] = norm_rope(v, None, 0.0, HK, 0, 1.0, 0, dtype)
    o = sdpa(qr, kcache[:, :, :offset + L], vcache[:, :, :offset + L], D ** -0.5, L > 1, dtype)
    o = np.ascontiguousarray(np.transpose(o, (0, 2, 1, 3))).reshape(1, L, H * D)
    h = round_to(x.astype(np.float64) + proj(o, W["o_proj"]), dtype)
    hn = rms_norm(h, W["post_attention_layernorm"], eps, dtype)
    g = proj(hn, W["gate_proj"])
    u = proj(hn, W["up_proj"])
    d = proj(swiglu(g, u, dtype), W["down_proj"])
    return round_to(h.astype(np.float64) + d, dtype)


def qwen3_forward(ids, layers: list, embed, final_norm, cfg, offset: int, kcaches, vcaches,
                  dtype: str = "bfloat16"):
    """Embedding (dequantized rows) -> layers -> norm of the last position ->
    tied lm_head. Returns logits [1, 1, vocab] (values of T)."""
    wq, s, b = embed
    rows = np.asarray(ids).reshape(-1)
    q = unpack(wq[rows], cfg.bits).astype(np.float32)
    h = round_to(np.repeat(s[rows], cfg.group_size, 1) * q + np.repeat(b[rows], cfg.group_size, 1),
                 dtype)[None]
    for i, W in enumerate(layers):
        h = qwen3_layer(h, W, cfg, offset, kcaches[i], vcaches[i], dtype)
    hn = rms_norm(h[:, -1:], final_norm, cfg.rms_norm_eps, dtype)
    return qmm_factored(hn, wq, s, b, cfg.group_size, cfg.bits, dtype)


# ----------------------------------------------------------------------------
# LFM2 hybrid (config 5): the op streams of the reference's generated
# wrappers, examples/lfm2_5_1_2b_prefill/lfm2_5_1_2b_prefill_artifact/
# patch/wrappers.py (conv layers :38-106, attention layers :145-220)


def lfm2_mlp(hn, h, W: dict, cfg, dtype: str = "bfloat16"):
    """[qmm(w1), qmm(w3)] -> swiglu -> [qmm(w2), add] (wrappers.py:81-106)."""
    gs, bits = cfg.group_size, cfg.bits
    g = _qmm_auto(hn, W["w1"], gs, bits, dtype)
    u = _qmm_auto(hn, W["w3"], gs, bits, dtype)
    d = _qmm_auto(swiglu(g, u, dtype), W["w2"], gs, bits, dtype)
    return round_to(np.asarray(h, np.float64) + d, dtype)


def lfm2_conv_layer(x, W: dict, cfg, state, dtype: str = "bfloat16"):
    """Gated short-conv layer (wrappers.py:38-106): rms_norm(operator_norm) ->
    qmm(in_proj) -> split(3) = (B, C, x) -> B*x -> conv over
    concat(state or zeros, B*x) -> C*conv -> qmm(out_proj) + residual ->
    rms_norm(ffn_norm) -> MLP + residual. W["conv"] is the [D, 3] depthwise
    weight. Returns (layer output, new conv state)."""
    gs, bits, eps = cfg.group_size, cfg.bits, cfg.norm_eps
    xn = rms_norm(x, W["operator_norm"], eps, dtype)
    c, bx = split_gate(_qmm_auto(xn, W["in_proj"], gs, bits, dtype), dtype)
    y, new_state = shortconv(bx, c, W["conv"], state, dtype)
    h = round_to(np.asarray(x, np.float64) + _qmm_auto(y, W["out_proj"], gs, bits, dtype), dtype)
    hn = rms_norm(h, W["ffn_norm"], eps, dtype)
    return lfm2_mlp(hn, h, W, cfg, dtype), new_state


def lfm2_attn_layer(x, W: dict, cfg, offset: int, kcache, vcache, dtype: str = "bfloat16"):
    """Attention layer (wrappers.py:145-220): rms_norm(operator_norm) ->
    q/k/v qmm -> per-head rms_norm(q_layernorm / k_layernorm) -> rope (head
    dim, base rope_theta, offset) -> cache update -> causal sdpa (scale
    head_dim^-0.5) -> qmm(out_proj) + residual -> rms_norm(ffn_norm) -> MLP +
    residual. kcache/vcache [1, HK, cap, D] are written at [offset, offset+L)."""
    gs, bits, eps = cfg.group_size, cfg.bits, cfg.norm_eps
    H, HK, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    L = x.shape[1]
    xn = rms_norm(x, W["operator_norm"], eps, dtype)
    q = _qmm_auto(xn, W["q_proj"], gs, bits, dtype)
    k = _qmm_auto(xn, W["k_proj"], gs, bits, dtype)
    v = _qmm_auto(xn, W["v_proj"], gs, bits, dtype)
    qr = norm_rope(q, W["q_layernorm"], eps, H, D, cfg.rope_theta, offset, dtype)
    kcache[:, :, offset:offset + L] = norm_rope(k, W["k_layernorm"], eps, HK, D, cfg.rope_theta,
                                                offset, dtype)
    vcache[:, :, offset:offset + L] = norm_rope(v, None, 0.0, HK, 0, 1.0, 0, dtype)
    o = sdpa(qr, kcache[:, :, :offset + L], vcache[:, :, :offset + L], D ** -0.5, L > 1, dtype)
    o = np.ascontiguousarray(np.transpose(o, (0, 2, 1, 3))).reshape(1, L, H * D)
    h = round_to(np.asarray(x, np.float64) + _qmm_auto(o, W["out_proj"], gs, bits, dtype), dtype)
    hn = rms_norm(h, W["ffn_norm"], eps, dtype)
    return lfm2_mlp(hn, h, W, cfg, dtype)


def lfm2_layer_window(x, W: dict, cfg, kind: str, rows: int, dtype: str = "bfloat16"):
    """Output rows [L - rows, L) of one LFM2 layer over its whole input x
    [1, L, hidden] (fresh state, offset 0), computed on only what those rows
    read. A conv layer's row t reads input rows t-2..t (the 3-tap causal conv
    over B*x, wrappers.py:57-66; everything else is row-wise), so the window
    runs on rows + 2 input rows from a zero state and drops the two context
    rows. An attention layer's window attends to every earlier row: the keys
    and values of rows [0, L - rows) are the cache update of
    lfm2_attn_layer on those rows (row-wise: rms_norm, k/v qmm, k-norm + RoPE
    at offset 0), and the window runs as the next chunk at offset L - rows
    (mlx-lm's chunked prefill). The same values as lfm2_attn_layer /
    lfm2_conv_layer over the whole x, restricted to the window, bit for bit,
    when every projection sees more than 8 rows in both forms: _qmm_auto
    routes M <= 8 to the factored qmv (stitch.py:74-100), so a shorter window
    or key prefix would round its projections differently."""
    L = x.shape[1]
    s = L - rows
    if rows < 9 or rows > L or (kind != "conv" and 0 < s < 9):
        raise ValueError(f"window of {rows} rows over {L}: the window, and an attention "
                         "layer's key prefix, need more than 8 rows")
    if kind == "conv":
        y, _ = lfm2_conv_layer(x[:, max(s - 2, 0):], W, cfg, None, dtype)
        return y[:, min(s, 2):]
    gs, bits, eps = cfg.group_size, cfg.bits, cfg.norm_eps
    HK, D = cfg.num_key_value_heads, cfg.head_dim
    kc = np.zeros((1, HK, L, D), np.float32)
    vc = np.zeros_like(kc)
    if s > 0:
        xn = rms_norm(x[:, :s], W["operator_norm"], eps, dtype)
        kc[:, :, :s] = norm_rope(_qmm_auto(xn, W["k_proj"], gs, bits, dtype), W["k_layernorm"],
                                 eps, HK, D, cfg.rope_theta, 0, dtype)
        vc[:, :, :s] = norm_rope(_qmm_auto(xn, W["v_proj"], gs, bits, dtype), None, 0.0, HK, 0,
                                 1.0, 0, dtype)
    return lfm2_attn_layer(x[:, s:], W, cfg, s, kc, vc, dtype)
