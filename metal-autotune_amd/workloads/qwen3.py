"""Qwen3-4B-shaped decoder with 4-bit affine weights (benchmark configs 3 and 4).

The module tree mirrors mlx-lm's qwen3 model (model.embed_tokens,
model.layers[i].self_attn.{q,k,v,o}_proj / q_norm / k_norm,
model.layers[i].mlp.{gate,up,down}_proj, input_layernorm,
post_attention_layernorm, model.norm; tied embedding), so region wrappers
resolve weights by the dot paths the reference's generated wrappers use
(patch/wrappers.py:17-36 resolves 'self_attn.q_proj.weight' the same way).

``DecoderLayer.forward`` is the original op sequence, one library op per MLX
op (quantized_matmul, rms_norm, rope, sdpa, swiglu, adds) -- the analog of
the recorded op stream a generated wrapper replays. ``Qwen3LayerRegions`` is
the installed wrapper: it splices the reference-style region cuts through
``kernels.try_sized`` and falls back to the original ops when a spec's
fallback predicate fires (patch/wrappers.py:51-55 pattern):

  [qmm(o_proj), add, rms_norm(post_attention_layernorm)] -> residual_rmsnorm
  [qmm(gate), qmm(up), swiglu]                           -> dual_swiglu
  [qmm(down), add]                                       -> residual
  [qmm(q), qmm(k), qmm(v)]                               -> qkv (grouped3)
  reshape -> q_norm/k_norm -> transpose -> rope (+cache)  -> norm_rope_qkv

Where the qkv cut serves the call, the two last rows run as one launch
(``ops.qkv_norm_rope``: the prologue in the GEMM's epilogue, the same bits);
shapes the fused entry does not take run them as two.

``install_regions`` also links neighbouring layers: layer i's last cut
becomes [qmm(down), add, rms_norm(layer i+1's input_layernorm)], the same
region kind as the o_proj cut, and layer i+1 takes that normalized output
instead of normalizing its input again (one launch fewer per layer, same
bits).

Only the last position's logits are computed in prefill (the caller takes
logits[:, -1] before sampling; everything before it is dead work,
docs/measurement.md:74-83).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
from torch import nn

from autotuner_runtime import ops, regions
from autotuner_runtime.serve import SizedRegions
from autotuner_runtime.swap import install

from .quantize import random_quantized


@dataclass(frozen=True)
class Qwen3Config:
    hidden_size: int = 2560
    num_hidden_layers: int = 36
    num_attention_heads: int = 32
    num_key_value_heads: int = 8
    head_dim: int = 128
    intermediate_size: int = 9728
    vocab_size: int = 151936
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    group_size: int = 64
    bits: int = 4


class QuantizedLinear(nn.Module):
    def __init__(self, w, s, b, group_size: int, bits: int):
        super().__init__()
        self.register_buffer("weight", w)
        self.register_buffer("scales", s)
        self.register_buffer("biases", b)
        self.group_size, self.bits = group_size, bits

    def forward(self, x):
        return ops.quantized_matmul(x, self.weight, self.scales, self.biases,
                                    group_size=self.group_size, bits=self.bits)


class QuantizedEmbedding(QuantizedLinear):
    def forward(self, ids):
        return ops.quantized_embedding(ids, self.weight, self.scales, self.biases,
                                       self.group_size, self.bits)

    def as_linear(self, x):
        return ops.quantized_matmul(x, self.weight, self.scales, self.biases,
                                    group_size=self.group_size, bits=self.bits)


class RMSNorm(nn.Module):
    def __init__(self, weight, eps: float):
        super().__init__()
        self.register_buffer("weight", weight)
        self.eps = eps

    def forward(self, x):
        return ops.rms_norm(x, self.weight, self.eps)


class KVCache:
    """Preallocated [1, HK, max_len, D] keys/values; update_and_fetch writes rows
    [offset, offset + L) in place (the kernels write straight into it)."""

    def __init__(self, n_kv_heads, head_dim, max_len, device, dtype=torch.bfloat16):
        self.keys = torch.zeros((1, n_kv_heads, max_len, head_dim), device=device, dtype=dtype)
        self.values = torch.zeros_like(self.keys)
        self.offset = 0


class Attention(nn.Module):
    def __init__(self, cfg: Qwen3Config, mods: dict):
        super().__init__()
        self.cfg = cfg
        for k, v in mods.items():
            setattr(self, k, v)
        self.scale = 1.0 / math.sqrt(cfg.head_dim)

    def forward(self, x, cache: KVCache):
        c = self.cfg
        B, L, _ = x.shape
        q = self.q_proj(x)
        k = self.k_proj(x)
        v = self.v_proj(x)
        qr = ops.norm_rope(q, self.q_norm.weight, c.num_attention_heads, c.rms_norm_eps,
                           c.head_dim, c.rope_theta, cache.offset)
        ops.norm_rope(k, self.k_norm.weight, c.num_key_value_heads, c.rms_norm_eps, c.head_dim,
                      c.rope_theta, cache.offset, out=cache.keys, out_pos=cache.offset)
        ops.write_kv(v, c.num_key_value_heads, cache.values, cache.offset)
        o = ops.scaled_dot_product_attention(qr, cache.keys, cache.values, self.scale,
                                             "causal" if L > 1 else None,
                                             kv_len=cache.offset + L, out_layout=1)
        return self.o_proj(o.reshape(B, L, -1))


class MLP(nn.Module):
    def __init__(self, mods: dict):
        super().__init__()
        for k, v in mods.items():
            setattr(self, k, v)

    def forward(self, x):
        return self.down_proj(ops.swiglu(self.gate_proj(x), self.up_proj(x)))


class DecoderLayer(nn.Module):
    def __init__(self, cfg: Qwen3Config, attn: Attention, mlp: MLP, in_norm, post_norm):
        super().__init__()
        self.self_attn = attn
        self.mlp = mlp
        self.input_layernorm = in_norm
        self.post_attention_layernorm = post_norm

    def forward(self, x, cache: KVCache):
        h = x + self.self_attn(self.input_layernorm(x), cache)
        return h + self.mlp(self.post_attention_layernorm(h))


class Qwen3Inner(nn.Module):
    def __init__(self, embed, layers, norm):
        super().__init__()
        self.embed_tokens = embed
        self.layers = nn.ModuleList(layers)
        self.norm = norm


class Qwen3Model(nn.Module):
    def __init__(self, cfg: Qwen3Config, inner: Qwen3Inner):
        super().__init__()
        self.cfg = cfg
        self.model = inner

    def make_cache(self, max_len: int):
        dev = self.model.norm.weight.device
        return [KVCache(self.cfg.num_key_value_heads, self.cfg.head_dim, max_len, dev)
                for _ in self.model.layers]

    def forward(self, ids, caches, last_only: bool = True):
        """ids [1, L] int -> logits [1, 1 or L, vocab]; advances the caches."""
        h = self.model.embed_tokens(ids)
        for layer, cache in zip(self.model.layers, caches):
            h = layer(h, cache)
        for cache in caches:
            cache.offset += ids.shape[1]
        if last_only:
            h = h[:, -1:, :]
        return self.model.embed_tokens.as_linear(self.model.norm(h))


# ---------------------------------------------------------------------------
# region wrapper


def layer_specs(cfg: Qwen3Config, dtype: str = "bfloat16") -> dict:
    gs, bits = cfg.group_size, cfg.bits
    return {
        "qkv": regions.grouped3("qwen3_qkv_proj", dtype, gs, bits),
        "residual_rmsnorm": regions.residual_rmsnorm("qwen3_o_proj_add_norm", dtype, gs, bits,
                                                     cfg.rms_norm_eps),
        "dual_swiglu": regions.dual_swiglu("qwen3_gate_up_swiglu", dtype, gs, bits),
        "residual": regions.residual("qwen3_down_add", dtype, gs, bits),
    }


class NormHandoff:
    """The next layer's normalized input, made by the previous layer's last
    region together with that layer's output h. It is handed over only for
    that very tensor: a layer called with any other input normalizes it
    itself."""

    __slots__ = ("h", "hn")

    def __init__(self):
        self.h = self.hn = None

    def put(self, h, hn) -> None:
        self.h, self.hn = h, hn

    def take(self, x):
        h, hn = self.h, self.hn
        self.h = self.hn = None
        return hn if h is x else None


class Qwen3LayerRegions(SizedRegions):
    """The decoder layer with the region cuts spliced in (try_sized at the
    sizes each kernel serves, else the original ops). A spec missing from the
    table leaves its cut on the original ops."""

    KERNEL_IDS = ["qwen3_qkv_proj", "qwen3_o_proj_add_norm", "qwen3_gate_up_swiglu",
                  "qwen3_down_add"]

    def link(self, prev: NormHandoff | None = None, nxt=None) -> None:
        """prev: where the previous layer leaves this layer's normalized input;
        nxt: (the next layer's input RMSNorm, the [qmm(down), add, rms_norm]
        spec, the handoff to the next layer). Plain attributes, not submodules."""
        self.__dict__["_prev"] = prev
        self.__dict__["_next"] = nxt

    def forward(self, x, cache: KVCache):
        w = self.wrapped
        if not (x.dim() == 3 and x.dtype == torch.bfloat16 and x.is_cuda):
            return w(x, cache)
        attn, mlp = w.self_attn, w.mlp
        c = attn.cfg
        B, L, _ = x.shape
        prev = self.__dict__.get("_prev")
        xn = prev.take(x) if prev is not None else None
        if xn is None:
            xn = w.input_layernorm(x)
        projs = (attn.q_proj, attn.k_proj, attn.v_proj)
        ins = [xn] + [t for m in projs for t in (m.weight, m.scales, m.biases)]
        qr = None
        if self._serves("qkv", ins, L):
            # the q/k/v cut with the prologue below in its epilogue, the same
            # bits (None: shapes the fused entry does not take)
            qr = ops.qkv_norm_rope(xn, [(m.weight, m.scales, m.biases) for m in projs],
                                   attn.q_norm.weight, attn.k_norm.weight, c.num_attention_heads,
                                   c.num_key_value_heads, c.rms_norm_eps, c.head_dim,
                                   c.rope_theta, cache.offset, cache.keys, cache.values,
                                   cache.offset, c.group_size, c.bits)
        if qr is None:
            outs = self._try("qkv", ins, L)
            q, k, v = (m(xn) for m in projs) if outs is None else outs
            # q/k-norm + RoPE + the KV-cache update, one launch
            qr = ops.norm_rope_qkv(q, k, v, attn.q_norm.weight, attn.k_norm.weight,
                                   c.num_attention_heads, c.num_key_value_heads, c.rms_norm_eps,
                                   c.head_dim, c.rope_theta, cache.offset, cache.keys,
                                   cache.values, cache.offset)
        o = ops.scaled_dot_product_attention(qr, cache.keys, cache.values, attn.scale,
                                             "causal" if L > 1 else None,
                                             kv_len=cache.offset + L,
                                             out_layout=1).reshape(B, L, -1)
        op, pn = attn.o_proj, w.post_attention_layernorm
        outs = self._try("residual_rmsnorm", [o, op.weight, op.scales, op.biases, x, pn.weight], L)
        if outs is None:
            h = x + op(o)
            hn = pn(h)
        else:
            h, hn = outs
        g, u = mlp.gate_proj, mlp.up_proj
        outs = self._try("dual_swiglu",
                         [hn, g.weight, g.scales, g.biases, u.weight, u.scales, u.biases], L)
        act = ops.swiglu(g(hn), u(hn)) if outs is None else outs[0]
        d = mlp.down_proj
        nxt = self.__dict__.get("_next")
        if nxt is not None:
            norm, spec, handoff = nxt
            outs = self._try_spec(spec, [act, d.weight, d.scales, d.biases, h, norm.weight], L)
            if outs is not None:
                handoff.put(outs[0], outs[1])
                return outs[0]
        outs = self._try("residual", [act, d.weight, d.scales, d.biases, h], L)
        return h + d(act) if outs is None else outs[0]


def install_regions(model: Qwen3Model, link_layers: bool = True) -> list:
    """Swap the region wrapper in at every model.layers.i; returns the
    occupants. link_layers: each layer's down_proj cut also normalizes the
    next layer's input (NormHandoff)."""
    cfg = model.cfg
    specs = layer_specs(cfg)
    layers = list(model.model.layers)
    wrappers = [Qwen3LayerRegions(layer, specs) for layer in layers]
    if link_layers:
        spec = regions.residual_rmsnorm("qwen3_down_add_next_norm", "bfloat16", cfg.group_size,
                                        cfg.bits, cfg.rms_norm_eps)
        for i in range(len(layers) - 1):
            handoff = NormHandoff()
            wrappers[i].link(prev=wrappers[i].__dict__.get("_prev"),
                             nxt=(layers[i + 1].input_layernorm, spec, handoff))
            wrappers[i + 1].link(prev=handoff)
    return [install(model, f"model.layers.{i}", wr) for i, wr in enumerate(wrappers)]


# ---------------------------------------------------------------------------
# seeded random weights


def build(cfg: Qwen3Config = Qwen3Config(), seed: int = 0, device="cuda",
          num_layers: int | None = None) -> Qwen3Model:
    """Random-weight model: every projection N(0, 0.02) quantized with the build's
    affine rule; norm weights 1 + 0.1 N(0, 1) in bf16. Deterministic per seed."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    gs, bits, H, D = cfg.group_size, cfg.bits, cfg.hidden_size, cfg.head_dim

    def ql(n, k):
        return QuantizedLinear(*random_quantized(n, k, gen, device, gs, bits), gs, bits)

    def norm(n):
        w = (1.0 + 0.1 * torch.randn(n, generator=gen, device=device)).to(torch.bfloat16)
        return RMSNorm(w, cfg.rms_norm_eps)

    layers = []
    for _ in range(cfg.num_hidden_layers if num_layers is None else num_layers):
        attn = Attention(cfg, {
            "q_proj": ql(cfg.num_attention_heads * D, H),
            "k_proj": ql(cfg.num_key_value_heads * D, H),
            "v_proj": ql(cfg.num_key_value_heads * D, H),
            "o_proj": ql(H, cfg.num_attention_heads * D),
            "q_norm": norm(D),
            "k_norm": norm(D),
        })
        mlp = MLP({"gate_proj": ql(cfg.intermediate_size, H), "up_proj": ql(cfg.intermediate_size, H),
                   "down_proj": ql(H, cfg.intermediate_size)})
        layers.append(DecoderLayer(cfg, attn, mlp, norm(H), norm(H)))
    embed = QuantizedEmbedding(*random_quantized(cfg.vocab_size, H, gen, device, gs, bits), gs, bits)
    return Qwen3Model(cfg, Qwen3Inner(embed, layers, norm(H)))


def tokens(seed: int, n: int, vocab: int, device="cuda") -> torch.Tensor:
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    return torch.randint(0, vocab, (1, n), generator=gen, dtype=torch.int64).to(device)
