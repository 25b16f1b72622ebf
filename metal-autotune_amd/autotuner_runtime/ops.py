"""Tensor-level ops on the gfx950 library: the library calls the reference's
regions splice around (mx.quantized_matmul, mx.dequantize, mx.fast.rms_norm,
mx.fast.rope, mx.fast.scaled_dot_product_attention, mlx-lm's swiglu and
quantized embedding, LFM2's short-conv) plus the fused region entry points.

Every function allocates its outputs with torch on the inputs' device and
launches on torch's current stream; none synchronizes. They run only on GPU
tensors (hip.lib() raises otherwise); there is no CPU path.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import hip


def _empty(shape, like: torch.Tensor, dtype=None) -> torch.Tensor:
    return torch.empty(shape, dtype=dtype or like.dtype, device=like.device)


def _qp(group_size: int, bits: int) -> dict:
    return {"group_size": group_size, "bits": bits}


# -- A1 ---------------------------------------------------------------------

def dequantize(w, scales, biases, group_size: int = 64, bits: int = 4) -> torch.Tensor:
    """mx.dequantize (affine): T(fma(s, q, b)) as [N, K] in the scales' dtype."""
    N, K = w.shape[0], w.shape[1] * 32 // bits
    out = _empty((N, K), scales)
    hip.b_dequant([w, scales, biases], [out], _qp(group_size, bits))
    return out


def quantized_embedding(ids, w, scales, biases, group_size: int = 64, bits: int = 4):
    """nn.QuantizedEmbedding: dequantized rows ids -> [*ids.shape, K]."""
    K = w.shape[1] * 32 // bits
    out = _empty((*ids.shape, K), scales)
    hip.b_gather_dequant([ids.contiguous(), w, scales, biases], [out], _qp(group_size, bits))
    return out


# -- A2-A4 and the qmm regions ---------------------------------------------

def quantized_matmul(x, w, scales, biases, transpose: bool = True, group_size: int = 64,
                     bits: int = 4, mode: str = "affine") -> torch.Tensor:
    """mx.quantized_matmul(x, w, scales, biases, transpose=True, group_size, bits,
    mode='affine') -> x @ dequant(w)^T."""
    if not transpose or mode != "affine":
        raise ValueError("only transpose=True, mode='affine' is covered (the MLX checkpoint layout)")
    y = _empty((*x.shape[:-1], w.shape[0]), x)
    hip.b_qmm([x.contiguous(), w, scales, biases], [y], _qp(group_size, bits))
    return y


def qmm_residual(x, w, scales, biases, resid, group_size=64, bits=4):
    """Region [qmm, add]: T(resid + T(x @ W^T))."""
    y = _empty((*x.shape[:-1], w.shape[0]), x)
    hip.b_qmm_residual([x.contiguous(), w, scales, biases, resid.contiguous()], [y],
                       _qp(group_size, bits))
    return y


def qmm_residual_rmsnorm(x, w, scales, biases, resid, norm_w, eps: float, group_size=64, bits=4):
    """Region [qmm, add, rms_norm] -> (h, rms_norm(h))."""
    shape = (*x.shape[:-1], w.shape[0])
    h, y = _empty(shape, x), _empty(shape, x)
    hip.b_qmm_residual_rmsnorm([x.contiguous(), w, scales, biases, resid.contiguous(), norm_w],
                               [h, y], {**_qp(group_size, bits), "eps": eps})
    return h, y


def qmm_split_gate(x, w, scales, biases, group_size=64, bits=4):
    """Region [qmm, split(3), mul] -> (C, T(B * x))."""
    shape = (*x.shape[:-1], w.shape[0] // 3)
    c, bx = _empty(shape, x), _empty(shape, x)
    hip.b_qmm_split_gate([x.contiguous(), w, scales, biases], [c, bx], _qp(group_size, bits))
    return c, bx


def qmm_dual(x, w1, s1, b1, w2, s2, b2, group_size=64, bits=4, swiglu: bool = False):
    """Region [qmm(w1), qmm(w3)] -> (x W1^T, x W3^T), or swiglu of the two."""
    shape = (*x.shape[:-1], w1.shape[0])
    p = {**_qp(group_size, bits), "act": hip.MI_ACT_SWIGLU if swiglu else hip.MI_ACT_NONE}
    ins = [x.contiguous(), w1, s1, b1, w2, s2, b2]
    if swiglu:
        y = _empty(shape, x)
        hip.b_qmm_dual(ins, [y], p)
        return y
    y1, y2 = _empty(shape, x), _empty(shape, x)
    hip.b_qmm_dual(ins, [y1, y2], p)
    return y1, y2


def qmm_grouped3(x, weights, group_size=64, bits=4):
    """Three projections of one x in one launch: ``weights`` is three
    (w, scales, biases) triples; returns the three x @ dequant(w)^T."""
    outs = [_empty((*x.shape[:-1], w.shape[0]), x) for w, _, _ in weights]
    ins = [x.contiguous()] + [t for triple in weights for t in triple]
    hip.b_qmm_grouped3(ins, outs, _qp(group_size, bits))
    return outs


# -- A5, A6 ----------------------------------------------------------------

def rms_norm(x, weight, eps: float) -> torch.Tensor:
    """mx.fast.rms_norm over the last axis."""
    x = x.contiguous()
    y = torch.empty_like(x)
    hip.b_rms_norm([x, weight], [y], {"eps": eps})
    return y


def norm_rope(x, weight, n_heads: int, eps: float, dims: int, base: float, offset: int = 0,
              traditional: bool = False, scale: float = 1.0, out: torch.Tensor | None = None,
              out_pos: int = 0) -> torch.Tensor:
    """reshape(B, L, H, D) -> rms_norm(weight) (skipped if None) -> transpose(0,2,1,3)
    -> mx.fast.rope(dims, traditional, base, scale, offset). With ``out`` (a
    [B, H, cap, D] cache) the rows land at [out_pos, out_pos + L) in place."""
    x = x.contiguous()
    B, L, HD = x.shape
    D = HD // n_heads
    if out is None:
        out = _empty((B, n_heads, L, D), x)
        cap, pos = L, 0
    else:
        if not out.is_contiguous() or out.shape[0] != B or out.shape[1] != n_heads or out.shape[3] != D:
            raise ValueError(f"cache target {tuple(out.shape)} does not hold {(B, n_heads, '*', D)}")
        cap, pos = out.shape[2], out_pos
    if weight is not None and (tuple(weight.shape) != (D,) or weight.dtype != x.dtype):
        raise ValueError(f"norm weight must be {x.dtype} [{D}]")
    hip._require_gpu(x)
    hip._check(hip.lib().mi_norm_rope(
        x.data_ptr(), None if weight is None else weight.data_ptr(), out.data_ptr(), B, L,
        n_heads, D, HD, float(eps), int(dims), int(traditional), float(base), float(scale),
        int(offset), cap, pos, hip._dt(x), hip._stream(x)), "norm_rope")
    return out


def norm_rope_qkv(q, k, v, q_norm, k_norm, n_heads: int, n_kv_heads: int, eps: float, dims: int,
                  base: float, offset: int, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  cache_pos: int, traditional: bool = False, scale: float = 1.0) -> torch.Tensor:
    """The attention prologue in one launch: q -> rms_norm -> rope -> [B, H, L, D]
    (returned); k -> rms_norm -> rope and v -> transpose, written into the
    caches at rows [cache_pos, cache_pos + L). Equal bit for bit to three
    norm_rope calls. q, k, v may be row-strided views ([B, L, H*D] slices)."""
    B, L, _ = q.shape
    D = q.shape[-1] // n_heads
    for t, h in ((k, n_kv_heads), (v, n_kv_heads)):
        if t.shape[:2] != (B, L) or t.shape[-1] != h * D or t.dtype != q.dtype:
            raise ValueError("q, k and v must share batch, length, head dim and dtype")
    for t in (q, k, v):
        if t.stride(-1) != 1 or t.stride(0) != L * t.stride(1):
            raise ValueError("q, k, v rows must be unit-stride with a uniform row stride")
    for c in (k_cache, v_cache):
        if (not c.is_contiguous() or c.shape[0] != B or c.shape[1] != n_kv_heads
                or c.shape[3] != D or c.dtype != q.dtype):
            raise ValueError(f"cache {tuple(c.shape)} does not hold {(B, n_kv_heads, '*', D)}")
    for wt in (q_norm, k_norm):
        if tuple(wt.shape) != (D,) or wt.dtype != q.dtype:
            raise ValueError(f"norm weight must be {q.dtype} [{D}]")
    out = _empty((B, n_heads, L, D), q)
    hip._require_gpu(q)
    hip._check(hip.lib().mi_norm_rope_qkv(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), q.stride(1), k.stride(1), v.stride(1),
        q_norm.data_ptr(), k_norm.data_ptr(), out.data_ptr(), k_cache.data_ptr(),
        v_cache.data_ptr(), B, L, n_heads, n_kv_heads, D, float(eps), int(dims),
        int(traditional), float(base), float(scale), int(offset), k_cache.shape[2],
        int(cache_pos), hip._dt(q), hip._stream(q)), "norm_rope_qkv")
    return out


def qkv_norm_rope(x, weights, q_norm, k_norm, n_heads: int, n_kv_heads: int, eps: float,
                  dims: int, base: float, offset: int, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, cache_pos: int, group_size: int = 64, bits: int = 4,
                  traditional: bool = False, scale: float = 1.0) -> torch.Tensor | None:
    """The q/k/v projections and the attention prologue in one launch:
    ``norm_rope_qkv(*qmm_grouped3(x, weights), ...)`` bit for bit, without
    writing q, k and v (patch/wrappers.py:156-176). ``weights`` is the (w,
    scales, biases) triples of q, k and v. Returns q_out [B, Hq, L, D] (k and v
    go into the caches at rows [cache_pos, cache_pos + L)), or None when the
    fused entry does not cover these shapes -- the caller then runs the two
    ops."""
    if x.dim() != 3:
        raise ValueError(f"x must be [B, L, K], got {tuple(x.shape)}")
    B, L, _ = x.shape
    p = _qp(group_size, bits)
    Ns = [hip._qmm_dims(x, w, s, b, p)[1] for w, s, b in weights]
    if Ns[0] % n_heads or Ns[1] % n_kv_heads or Ns[2] != Ns[1]:
        raise ValueError(f"projection widths {Ns} do not split into {n_heads} / {n_kv_heads} heads")
    D = Ns[0] // n_heads
    if Ns[1] // n_kv_heads != D:
        raise ValueError("q and k/v heads must share a head dim")
    for c in (k_cache, v_cache):
        if (not c.is_contiguous() or c.dim() != 4 or c.shape[0] != B
                or c.shape[1] != n_kv_heads or c.shape[3] != D or c.dtype != x.dtype):
            raise ValueError(f"cache {tuple(c.shape)} does not hold {(B, n_kv_heads, '*', D)}")
    for wt in (q_norm, k_norm):
        if tuple(wt.shape) != (D,) or wt.dtype != x.dtype or not wt.is_contiguous():
            raise ValueError(f"norm weight must be contiguous {x.dtype} [{D}]")
    hip._require_gpu(x)
    x = x.contiguous()
    hip._contig(*[t for triple in weights for t in triple])
    dt = hip._act_dtype(x, weights[0][1])
    out = _empty((B, n_heads, L, D), x)
    ptrs = ctypes.c_void_p * 3
    status = hip.lib().mi_qmm_affine_qkv_norm_rope(
        x.data_ptr(), ptrs(*[w.data_ptr() for w, _, _ in weights]),
        ptrs(*[s.data_ptr() for _, s, _ in weights]), ptrs(*[b.data_ptr() for _, _, b in weights]),
        q_norm.data_ptr(), k_norm.data_ptr(), out.data_ptr(), k_cache.data_ptr(),
        v_cache.data_ptr(), B, L, n_heads, n_kv_heads, D, x.shape[-1], group_size, bits,
        float(eps), int(dims), int(traditional), float(base), float(scale), int(offset),
        k_cache.shape[2], int(cache_pos), dt, hip._stream(x))
    if status == hip.MI_ERR_UNSUPPORTED:
        return None
    hip._check(status, "qkv_norm_rope")
    return out


def rope(x, dims: int, traditional: bool = False, base: float = 10000.0, scale: float = 1.0,
         offset: int = 0) -> torch.Tensor:
    """mx.fast.rope on [..., L, D] (the position axis is -2)."""
    x = x.contiguous()
    L, D = x.shape[-2], x.shape[-1]
    lead = x.numel() // (L * D) if L * D else 0
    flat = x.reshape(lead, L, D)  # one "head" per leading index: [B', L, 1*D]
    out = norm_rope(flat, None, 1, 0.0, dims, base, offset, traditional, scale)
    return out.reshape(x.shape)


def write_kv(v, n_heads: int, cache: torch.Tensor, pos: int) -> None:
    """The value half of a KV cache's update_and_fetch: reshape(B, L, H, D),
    transpose(0, 2, 1, 3), written into cache rows [pos, pos + L)."""
    norm_rope(v, None, n_heads, 0.0, 0, 1.0, 0, out=cache, out_pos=pos)


# -- A7 --------------------------------------------------------------------

def scaled_dot_product_attention(q, k, v, scale: float, mask: str | None = "causal",
                                 kv_len: int | None = None, out_layout: int = 0):
    """mx.fast.scaled_dot_product_attention(q, k, v, scale, mask='causal'|None).
    q [B, H, Lq, D]; k, v [B, HK, cap, D] with the first ``kv_len`` rows valid
    (default: all). out_layout 1 returns [B, Lq, H, D] (the transpose before
    o_proj, fused)."""
    if mask not in ("causal", None):
        raise ValueError("mask must be 'causal' or None")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    B, H, Lq, D = q.shape
    HK, cap = k.shape[1], k.shape[2]
    Lk = cap if kv_len is None else int(kv_len)
    o = _empty((B, H, Lq, D) if out_layout == 0 else (B, Lq, H, D), q)
    hip._require_gpu(q)
    if tuple(v.shape) != tuple(k.shape) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("k and v must match each other and q's dtype")
    hip._check(hip.lib().mi_sdpa(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H, HK,
                                 Lq, Lk, D, cap, float(scale), int(mask == "causal"),
                                 int(out_layout), hip._dt(q), hip._stream(q)), "sdpa")
    return o


# -- A8-A10, A12 -------------------------------------------------------------

def swiglu(g, u) -> torch.Tensor:
    """mlx_lm.models.activations.swiglu(gate, up) = silu(gate) * up."""
    g, u = g.contiguous(), u.contiguous()
    y = torch.empty_like(g)
    hip.b_swiglu([g, u], [y], {})
    return y


def shortconv(bx, c, w, state=None):
    """LFM2 short-conv core -> (T(c * conv(concat(state, bx))), new state [B, 2, D])."""
    bx, c = bx.contiguous(), c.contiguous()
    out = torch.empty_like(bx)
    st = _empty((bx.shape[0], 2, bx.shape[2]), bx)
    ins = [bx, c, w.contiguous()] + ([state.contiguous()] if state is not None else [])
    hip.b_shortconv(ins, [out, st], {})
    return out, st


def linear_f32(x, w, bias=None, gelu: bool = False) -> torch.Tensor:
    """nn.Linear in fp32 (mx.addmm(b, x, W^T)), optionally followed by exact GELU."""
    x = x.contiguous()
    y = _empty((*x.shape[:-1], w.shape[0]), x)
    ins = [x, w.contiguous()] + ([bias.contiguous()] if bias is not None else [])
    hip.b_linear_f32(ins, [y], {"act": hip.MI_ACT_GELU if gelu else hip.MI_ACT_NONE})
    return y


def gelu_mlp_f32(x, w1, b1, w2, b2) -> torch.Tensor:
    """Config 1's tiny MLP in one launch: gelu(x W1^T + b1) W2^T + b2 (fp32)."""
    x = x.contiguous()
    y = _empty((x.shape[0], w2.shape[0]), x)
    hip.b_gelu_mlp_f32([x, w1.contiguous(), b1.contiguous(), w2.contiguous(), b2.contiguous()],
                       [y], {})
    return y


def argmax(x, split: bool = True) -> torch.Tensor:
    """Greedy token: argmax over the last axis (lowest index on ties) as int32.
    split: each row over many workgroups (default) or one workgroup per row;
    the result is the same."""
    x = x.contiguous()
    o = _empty(x.shape[:-1], x, torch.int32)
    hip.b_argmax([x], [o], {"split": split})
    return o


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)
