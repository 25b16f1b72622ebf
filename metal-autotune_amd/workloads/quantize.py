"""The build's affine quantizer on torch tensors (CPU or GPU), for model set-up.

Per group of ``group_size`` values along K: s = (max - min) / (2^bits - 1),
b = min, both rounded to the activation dtype; q = clip(round((w - b) / s)),
packed LSB-first into uint32 words (MLX's layout). This is the build's own
rule, not mx.quantize (whose exact scale/bias choice only an MLX import could
pin); its outputs are the INPUTS of the quantized-matmul path, so it enters no
parity claim. It is not on the measured path.
"""

from __future__ import annotations

import torch


def pack(q: torch.Tensor, bits: int) -> torch.Tensor:
    """int codes [N, K] -> uint32 [N, K*bits/32], value j of a word at bit j*bits."""
    N, K = q.shape
    per = 32 // bits
    q = q.to(torch.int64).reshape(N, K // per, per)
    shifts = torch.arange(per, device=q.device, dtype=torch.int64) * bits
    words = (q << shifts).sum(dim=-1)
    # the same 32 bits as a signed int32 (exact, no overflowing conversion), viewed as uint32
    words = torch.where(words >= 2 ** 31, words - 2 ** 32, words)
    return words.to(torch.int32).view(torch.uint32)


def quantize_affine(w: torch.Tensor, group_size: int = 64, bits: int = 4,
                    dtype: torch.dtype = torch.bfloat16):
    """-> (packed uint32 [N, K*bits/32], scales [N, K/gs], biases [N, K/gs]) in dtype."""
    w = w.to(torch.float32)
    N, K = w.shape
    if K % group_size:
        raise ValueError("K must be a multiple of group_size")
    levels = (1 << bits) - 1
    g = w.reshape(N, K // group_size, group_size)
    lo = g.amin(dim=-1)
    hi = g.amax(dim=-1)
    s = ((hi - lo) / levels).to(dtype)
    b = lo.to(dtype)
    sf = s.to(torch.float32)
    safe = torch.where(sf == 0, torch.ones_like(sf), sf)
    q = torch.round((g - b.to(torch.float32)[..., None]) / safe[..., None])
    q = q.clamp_(0, levels).reshape(N, K)
    return pack(q, bits), s.contiguous(), b.contiguous()


def random_quantized(N: int, K: int, gen: torch.Generator, device, group_size=64, bits=4,
                     dtype=torch.bfloat16, std: float = 0.02):
    """A seeded N(0, std) weight quantized with the build's rule."""
    w = torch.randn((N, K), generator=gen, device=device, dtype=torch.float32) * std
    out = quantize_affine(w, group_size, bits, dtype)
    del w
    return out
