"""Exact tensor comparison: equal shapes, dtypes and bytes, so signed zeros and
NaN payloads count (the reference's exact.py:5-10, on torch tensors)."""

import torch


def bitwise_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    if tuple(a.shape) != tuple(b.shape) or a.dtype != b.dtype:
        return False
    if a.numel() == 0:
        return True
    ab = a.detach().contiguous().reshape(-1).view(torch.uint8)
    bb = b.detach().contiguous().reshape(-1).view(torch.uint8)
    if ab.device != bb.device:
        bb = bb.to(ab.device)
    return bool(torch.equal(ab, bb))
