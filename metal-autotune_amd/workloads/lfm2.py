"""LFM2-1.2B-shaped hybrid model with 4- or 8-bit affine weights (benchmark config 5).

The module tree follows mlx-lm's lfm2 model as the reference's generated
wrappers address it (examples/lfm2_5_1_2b_prefill/lfm2_5_1_2b_prefill_artifact/
patch/wrappers.py:17-36,114-142): model.embed_tokens, model.layers[i] with
operator_norm, ffn_norm, feed_forward.{w1,w2,w3}, and either
conv.{in_proj,conv,out_proj} (gated short-conv layers) or
self_attn.{q,k,v,out}_proj / q_layernorm / k_layernorm (attention layers);
model.embedding_norm; tied embedding as the lm_head.

``ConvLayer.forward`` / ``AttnLayer.forward`` are the original op streams,
one library op per MLX op (wrappers.py:38-106 and :145-220): quantized_matmul,
rms_norm, split + multiply, the short convolution over concat(state, B*x),
rope, sdpa, swiglu, adds. ``Lfm2ConvRegions`` / ``Lfm2AttnRegions`` are the
installed wrappers: the reference's cuts go through ``kernels.try_sized`` and
fall back to the original ops when a spec's predicate fires:

  [qmm(in_proj), split(3), mul]         -> split_gate         (wrappers.py:47-55)
  [qmm(out_proj), add, rms_norm]        -> residual_rmsnorm   (wrappers.py:67-80)
  [qmm(w1), qmm(w3)] + swiglu           -> dual_swiglu        (wrappers.py:81-96)
  [qmm(w2), add]                        -> residual           (wrappers.py:97-106)
  [qmm(q), qmm(k), qmm(v)]              -> grouped3           (wrappers.py:156-164)
  q/k layernorm + rope + cache update   -> norm_rope_qkv      (wrappers.py:165-176)

(the last two as one launch, ``ops.qkv_norm_rope``, where the qkv cut serves
the call and the fused entry takes the shape: from 512 tokens)

The reference's wrappers take the kernel path only for a fresh cache (conv
state None, attention offset 0, wrappers.py:34,148); these kernels take the
cache offset and conv state as inputs, so the region path also serves chunked
prefill and decode.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
from torch import nn

from autotuner_runtime import ops, regions
from autotuner_runtime.serve import SizedRegions
from autotuner_runtime.swap import ReplayWrapper, install

from .qwen3 import KVCache, QuantizedEmbedding, QuantizedLinear, RMSNorm
from .quantize import random_quantized


@dataclass(frozen=True)
class Lfm2Config:
    hidden_size: int = 2048
    num_hidden_layers: int = 16
    num_attention_heads: int = 32
    num_key_value_heads: int = 8
    intermediate_size: int = 8192
    vocab_size: int = 65536
    norm_eps: float = 1e-5
    rope_theta: float = 1e6
    conv_L_cache: int = 3
    full_attn_idxs: tuple = field(default=(2, 5, 8, 10, 12, 14))
    group_size: int = 64
    bits: int = 4

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads


class ConvCache:
    """The short-conv state: the last two rows of concat(state, B*x) [1, 2, D]
    (None before the first chunk, which convolves against zeros)."""

    def __init__(self):
        self.state = None
        self.offset = 0


class ShortConv(nn.Module):
    def __init__(self, mods: dict, conv_weight: torch.Tensor):
        super().__init__()
        for k, v in mods.items():
            setattr(self, k, v)
        self.conv = nn.Module()
        self.conv.register_buffer("weight", conv_weight)  # [D, 3, 1], mx.conv1d layout


class MLP(nn.Module):
    def __init__(self, mods: dict):
        super().__init__()
        for k, v in mods.items():
            setattr(self, k, v)

    def forward(self, x):
        return self.w2(ops.swiglu(self.w1(x), self.w3(x)))


class Attention(nn.Module):
    def __init__(self, cfg: Lfm2Config, mods: dict):
        super().__init__()
        self.cfg = cfg
        for k, v in mods.items():
            setattr(self, k, v)
        self.scale = 1.0 / math.sqrt(cfg.head_dim)


class ConvLayer(nn.Module):
    """operator_norm -> gated short-conv -> residual; ffn_norm -> SwiGLU MLP -> residual."""

    def __init__(self, cfg: Lfm2Config, conv: ShortConv, mlp: MLP, op_norm, ffn_norm):
        super().__init__()
        self.cfg = cfg
        self.conv = conv
        self.feed_forward = mlp
        self.operator_norm = op_norm
        self.ffn_norm = ffn_norm

    def forward(self, x, cache: ConvCache):
        c = self.conv
        xn = self.operator_norm(x)
        y = c.in_proj(xn)
        D = y.shape[-1] // 3
        Bg, Cg, xg = y[..., :D], y[..., D:2 * D], y[..., 2 * D:]
        bx = Bg * xg
        conv_out, cache.state = ops.shortconv(bx, Cg, c.conv.weight.reshape(D, 3), cache.state)
        h = x + c.out_proj(conv_out)
        return h + self.feed_forward(self.ffn_norm(h))


class AttnLayer(nn.Module):
    """operator_norm -> GQA attention (q/k layernorm, rope) -> residual; MLP."""

    def __init__(self, cfg: Lfm2Config, attn: Attention, mlp: MLP, op_norm, ffn_norm):
        super().__init__()
        self.self_attn = attn
        self.feed_forward = mlp
        self.operator_norm = op_norm
        self.ffn_norm = ffn_norm

    def forward(self, x, cache: KVCache):
        a = self.self_attn
        c = a.cfg
        B, L, _ = x.shape
        xn = self.operator_norm(x)
        q, k, v = a.q_proj(xn), a.k_proj(xn), a.v_proj(xn)
        qr = ops.norm_rope(q, a.q_layernorm.weight, c.num_attention_heads, c.norm_eps,
                           c.head_dim, c.rope_theta, cache.offset)
        ops.norm_rope(k, a.k_layernorm.weight, c.num_key_value_heads, c.norm_eps, c.head_dim,
                      c.rope_theta, cache.offset, out=cache.keys, out_pos=cache.offset)
        ops.write_kv(v, c.num_key_value_heads, cache.values, cache.offset)
        o = ops.scaled_dot_product_attention(qr, cache.keys, cache.values, a.scale,
                                             "causal" if L > 1 else None,
                                             kv_len=cache.offset + L, out_layout=1)
        h = x + a.out_proj(o.reshape(B, L, -1))
        return h + self.feed_forward(self.ffn_norm(h))


class Lfm2Inner(nn.Module):
    def __init__(self, embed, layers, norm):
        super().__init__()
        self.embed_tokens = embed
        self.layers = nn.ModuleList(layers)
        self.embedding_norm = norm


class Lfm2Model(nn.Module):
    def __init__(self, cfg: Lfm2Config, inner: Lfm2Inner):
        super().__init__()
        self.cfg = cfg
        self.model = inner

    def make_cache(self, max_len: int):
        """A KV cache per attention layer and a conv state per conv layer."""
        dev = self.model.embedding_norm.weight.device
        c = self.cfg
        out = []
        for layer in self.model.layers:
            base = layer.wrapped if isinstance(layer, ReplayWrapper) else layer
            out.append(KVCache(c.num_key_value_heads, c.head_dim, max_len, dev)
                       if isinstance(base, AttnLayer) else ConvCache())
        return out

    def forward(self, ids, caches, last_only: bool = True):
        """ids [1, L] -> logits [1, 1 or L, vocab]; advances the caches."""
        h = self.model.embed_tokens(ids)
        for layer, cache in zip(self.model.layers, caches):
            h = layer(h, cache)
        for cache in caches:
            cache.offset += ids.shape[1]
        if last_only:
            h = h[:, -1:, :]
        return self.model.embed_tokens.as_linear(self.model.embedding_norm(h))

    def prefill(self, ids, caches, chunk: int = 2048):
        """mlx-lm's chunked prefill: the prompt in pieces of at most ``chunk``
        tokens through the same caches; returns the last position's logits."""
        logits = None
        for s in range(0, ids.shape[1], chunk):
            logits = self.forward(ids[:, s:s + chunk], caches)
        return logits


# ---------------------------------------------------------------------------
# region wrappers


def layer_specs(cfg: Lfm2Config, dtype: str = "bfloat16") -> dict:
    gs, bits = cfg.group_size, cfg.bits
    return {
        "split_gate": regions.split_gate("lfm2_in_proj_split_gate", dtype, gs, bits),
        "qkv": regions.grouped3("lfm2_qkv_proj", dtype, gs, bits),
        "residual_rmsnorm": regions.residual_rmsnorm("lfm2_out_proj_add_norm", dtype, gs, bits,
                                                     cfg.norm_eps),
        "dual_swiglu": regions.dual_swiglu("lfm2_w1_w3_swiglu", dtype, gs, bits),
        "residual": regions.residual("lfm2_w2_add", dtype, gs, bits),
    }


def _mlp_regions(wr, mlp, hn, h, n):
    w1, w3 = mlp.w1, mlp.w3
    outs = wr._try("dual_swiglu",
                   [hn, w1.weight, w1.scales, w1.biases, w3.weight, w3.scales, w3.biases], n)
    act = ops.swiglu(w1(hn), w3(hn)) if outs is None else outs[0]
    w2 = mlp.w2
    outs = wr._try("residual", [act, w2.weight, w2.scales, w2.biases, h], n)
    return h + w2(act) if outs is None else outs[0]


def _out_proj_regions(wr, proj, o, x, ffn_norm, n):
    outs = wr._try("residual_rmsnorm",
                   [o, proj.weight, proj.scales, proj.biases, x, ffn_norm.weight], n)
    if outs is None:
        h = x + proj(o)
        return h, ffn_norm(h)
    return outs[0], outs[1]


class Lfm2ConvRegions(SizedRegions):
    """The short-conv layer with the region cuts spliced in (at the sizes each
    kernel serves)."""

    KERNEL_IDS = ["lfm2_in_proj_split_gate", "lfm2_out_proj_add_norm", "lfm2_w1_w3_swiglu",
                  "lfm2_w2_add"]

    def forward(self, x, cache: ConvCache):
        w = self.wrapped
        if not (x.dim() == 3 and x.dtype == torch.bfloat16 and x.is_cuda):
            return w(x, cache)
        c = w.conv
        L = x.shape[1]
        xn = w.operator_norm(x)
        p = c.in_proj
        outs = self._try("split_gate", [xn, p.weight, p.scales, p.biases], L)
        if outs is None:
            y = p(xn)
            D = y.shape[-1] // 3
            Cg, bx = y[..., D:2 * D], y[..., :D] * y[..., 2 * D:]
        else:
            Cg, bx = outs
        D = bx.shape[-1]
        conv_out, cache.state = ops.shortconv(bx, Cg, c.conv.weight.reshape(D, 3), cache.state)
        h, hn = _out_proj_regions(self, c.out_proj, conv_out, x, w.ffn_norm, L)
        return _mlp_regions(self, w.feed_forward, hn, h, L)


class Lfm2AttnRegions(SizedRegions):
    """The attention layer with the region cuts spliced in (at the sizes each
    kernel serves)."""

    KERNEL_IDS = ["lfm2_qkv_proj", "lfm2_out_proj_add_norm", "lfm2_w1_w3_swiglu", "lfm2_w2_add"]

    def forward(self, x, cache: KVCache):
        w = self.wrapped
        if not (x.dim() == 3 and x.dtype == torch.bfloat16 and x.is_cuda):
            return w(x, cache)
        a = w.self_attn
        c = a.cfg
        B, L, _ = x.shape
        xn = w.operator_norm(x)
        projs = (a.q_proj, a.k_proj, a.v_proj)
        ins = [xn] + [t for m in projs for t in (m.weight, m.scales, m.biases)]
        qr = None
        if self._serves("qkv", ins, L):
            # the q/k/v cut with the prologue below in its epilogue, the same
            # bits (None: shapes the fused entry does not take)
            qr = ops.qkv_norm_rope(xn, [(m.weight, m.scales, m.biases) for m in projs],
                                   a.q_layernorm.weight, a.k_layernorm.weight,
                                   c.num_attention_heads, c.num_key_value_heads, c.norm_eps,
                                   c.head_dim, c.rope_theta, cache.offset, cache.keys,
                                   cache.values, cache.offset, c.group_size, c.bits)
        if qr is None:
            outs = self._try("qkv", ins, L)
            q, k, v = (m(xn) for m in projs) if outs is None else outs
            qr = ops.norm_rope_qkv(q, k, v, a.q_layernorm.weight, a.k_layernorm.weight,
                                   c.num_attention_heads, c.num_key_value_heads, c.norm_eps,
                                   c.head_dim, c.rope_theta, cache.offset, cache.keys,
                                   cache.values, cache.offset)
        o = ops.scaled_dot_product_attention(qr, cache.keys, cache.values, a.scale,
                                             "causal" if L > 1 else None,
                                             kv_len=cache.offset + L,
                                             out_layout=1).reshape(B, L, -1)
        h, hn = _out_proj_regions(self, a.out_proj, o, x, w.ffn_norm, L)
        return _mlp_regions(self, w.feed_forward, hn, h, L)


def install_regions(model: Lfm2Model) -> list:
    """Swap the matching region wrapper in at every model.layers.i."""
    specs = layer_specs(model.cfg)
    out = []
    for i, layer in enumerate(model.model.layers):
        cls = Lfm2AttnRegions if isinstance(layer, AttnLayer) else Lfm2ConvRegions
        out.append(install(model, f"model.layers.{i}", cls(layer, specs)))
    return out


# ---------------------------------------------------------------------------
# seeded random weights


def build(cfg: Lfm2Config = Lfm2Config(), seed: int = 0, device="cuda",
          num_layers: int | None = None, layer_types: tuple | None = None) -> Lfm2Model:
    """Random-weight model: projections N(0, 0.02) quantized with the build's
    affine rule; norm weights 1 + 0.1 N(0, 1) and conv weights 0.3 N(0, 1) in
    bf16. ``layer_types`` ("conv" / "attn" per layer) overrides the config's
    pattern for partial models. Deterministic per seed."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    gs, bits, H, Dh = cfg.group_size, cfg.bits, cfg.hidden_size, cfg.head_dim

    def ql(n, k):
        return QuantizedLinear(*random_quantized(n, k, gen, device, gs, bits), gs, bits)

    def norm(n):
        w = (1.0 + 0.1 * torch.randn(n, generator=gen, device=device)).to(torch.bfloat16)
        return RMSNorm(w, cfg.norm_eps)

    def mlp():
        return MLP({"w1": ql(cfg.intermediate_size, H), "w3": ql(cfg.intermediate_size, H),
                    "w2": ql(H, cfg.intermediate_size)})

    n = cfg.num_hidden_layers if num_layers is None else num_layers
    types = layer_types or tuple("attn" if i in cfg.full_attn_idxs else "conv" for i in range(n))
    layers = []
    for kind in types:
        if kind == "attn":
            attn = Attention(cfg, {
                "q_proj": ql(cfg.num_attention_heads * Dh, H),
                "k_proj": ql(cfg.num_key_value_heads * Dh, H),
                "v_proj": ql(cfg.num_key_value_heads * Dh, H),
                "out_proj": ql(H, cfg.num_attention_heads * Dh),
                "q_layernorm": norm(Dh),
                "k_layernorm": norm(Dh),
            })
            layers.append(AttnLayer(cfg, attn, mlp(), norm(H), norm(H)))
        else:
            cw = (0.3 * torch.randn((H, cfg.conv_L_cache, 1), generator=gen, device=device))
            conv = ShortConv({"in_proj": ql(3 * H, H), "out_proj": ql(H, H)}, cw.to(torch.bfloat16))
            layers.append(ConvLayer(cfg, conv, mlp(), norm(H), norm(H)))
    embed = QuantizedEmbedding(*random_quantized(cfg.vocab_size, H, gen, device, gs, bits), gs, bits)
    return Lfm2Model(cfg, Lfm2Inner(embed, layers, norm(H)))
