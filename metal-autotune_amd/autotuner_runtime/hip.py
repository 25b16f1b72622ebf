"""ctypes binding of the gfx950 library (libmiqmm.so, C ABI in include/mi_qmm.h).

This is the backend under ``kernels.LoadedKernel`` and ``ops``: the analog of
the reference's ``mx.fast.metal_kernel`` dispatch (kernels.py:128-137,
212-220). There is no other backend and no CPU fallback: if the library is not
built, or no GPU is visible, every call raises RuntimeError.

Each C entry point has a binding here that takes the region's input tensors,
the runtime-allocated output tensors and the scalar parameters, checks shapes
and dtypes (ValueError on a mismatch, as the reference raises ValueError for
shapes a kernel does not cover), and launches on torch's current stream.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
import threading
from pathlib import Path
from typing import Callable

import torch

PKG = Path(__file__).resolve().parent.parent
LIB_PATH = Path(os.environ.get("MI_QMM_LIB", PKG / "libmiqmm.so"))
ABI_VERSION = 6

MI_F32, MI_F16, MI_BF16 = 0, 1, 2
MI_OK, MI_ERR_ARG, MI_ERR_UNSUPPORTED, MI_ERR_LAUNCH = 0, 1, 2, 3
MI_ACT_NONE, MI_ACT_SWIGLU, MI_ACT_GELU = 0, 1, 2

_DT = {torch.float32: MI_F32, torch.float16: MI_F16, torch.bfloat16: MI_BF16}

_P, _I64, _I, _F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
# symbol -> argtypes (restype int unless noted); the order of include/mi_qmm.h
SIGNATURES: dict[str, list] = {
    "mi_abi_version": [],
    "mi_last_error": [],
    "mi_affine_dequant": [_P, _P, _P, _P, _I64, _I64, _I, _I, _I, _P],
    "mi_affine_gather_dequant": [_P, _I64, _I, _P, _P, _P, _P, _I64, _I64, _I, _I, _I, _P],
    "mi_qmm_affine": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _I, _P],
    "mi_qmm_affine_residual": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _I, _P],
    "mi_qmm_affine_residual_rmsnorm": [_P, _P, _P, _P, _P, _P, _F, _P, _P, _I64, _I64, _I64,
                                       _I, _I, _I, _P],
    "mi_qmm_workspace_bytes": [_I64, _I64, _I64, _I, _I, _I],
    "mi_qmm_affine_ws": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _I, _P, _I64, _P],
    "mi_qmm_affine_residual_ws": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _I, _P,
                                  _I64, _P],
    "mi_qmm_affine_residual_rmsnorm_ws": [_P, _P, _P, _P, _P, _P, _F, _P, _P, _I64, _I64,
                                          _I64, _I, _I, _I, _P, _I64, _P],
    "mi_qmm_affine_split_gate": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _I, _P],
    "mi_qmm_affine_dual": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _I,
                           _I, _P],
    "mi_qmm_affine_grouped3": [_P, _P, _P, _P, _P, _I64, _P, _I64, _I, _I, _I, _P],
    "mi_rms_norm": [_P, _P, _P, _I64, _I64, _F, _I, _P],
    "mi_norm_rope": [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _I, _I, _F, _F, _I64, _I64,
                     _I64, _I, _P],
    "mi_norm_rope_qkv": [_P, _P, _P, _I64, _I64, _I64, _P, _P, _P, _P, _P, _I64, _I64, _I64,
                         _I64, _I64, _F, _I, _I, _F, _F, _I64, _I64, _I64, _I, _P],
    "mi_qmm_affine_qkv_norm_rope": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                    _I64, _I64, _I, _I, _F, _I, _I, _F, _F, _I64, _I64, _I64,
                                    _I, _P],
    "mi_sdpa": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F, _I, _I, _I, _P],
    "mi_swiglu": [_P, _P, _P, _I64, _I, _P],
    "mi_shortconv": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _P],
    "mi_linear_f32": [_P, _P, _P, _P, _I64, _I64, _I64, _I, _P],
    "mi_gelu_mlp_f32_workspace_bytes": [_I64, _I64, _I64, _I64],
    "mi_gelu_mlp_f32": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _P],
    "mi_argmax_workspace_bytes": [_I64, _I64],
    "mi_argmax": [_P, _P, _I64, _I64, _I, _P, _I64, _P],
    "mi_argmax_noalloc": [_P, _P, _I64, _I64, _I, _P],
}
RESTYPES = {"mi_last_error": ctypes.c_char_p, "mi_argmax_workspace_bytes": ctypes.c_int64,
            "mi_gelu_mlp_f32_workspace_bytes": ctypes.c_int64,
            "mi_qmm_workspace_bytes": ctypes.c_int64}

_lock = threading.Lock()
_lib = None


def library_path() -> Path:
    return LIB_PATH


def lib():
    """The loaded library; RuntimeError if it is not built or no GPU is visible."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build() "
                               "(the HIP library is the only backend)")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = argtypes
            fn.restype = RESTYPES.get(name, ctypes.c_int)
        if L.mi_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH}: ABI {L.mi_abi_version()} != {ABI_VERSION}")
        _lib = L
    return _lib


def exported_symbols() -> list[str]:
    """Every SIGNATURES symbol the library exports (no device needed)."""
    L = ctypes.CDLL(str(LIB_PATH))
    return [name for name in SIGNATURES if hasattr(L, name)]


def _require_gpu(t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise RuntimeError("the HIP library runs on GPU tensors only (got a CPU tensor); "
                           "there is no CPU fallback")


def _check(status: int, what: str) -> None:
    if status == MI_OK:
        return
    msg = lib().mi_last_error().decode(errors="replace")
    if status in (MI_ERR_ARG, MI_ERR_UNSUPPORTED):
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _dt(t: torch.Tensor) -> int:
    code = _DT.get(t.dtype)
    if code is None:
        raise ValueError(f"unsupported dtype {t.dtype}")
    return code


def _contig(*ts) -> None:
    for t in ts:
        if t is not None and not t.is_contiguous():
            raise ValueError("the HIP entry points take row-contiguous arrays")


def _quant(w: torch.Tensor, s: torch.Tensor, b: torch.Tensor, bits: int, gs: int):
    """(N, K) of a packed weight with its scales/biases (stitch.py:103-123)."""
    if w.dtype not in (torch.uint32, torch.int32) or w.dim() != 2:
        raise ValueError(f"packed weights must be a 2-d uint32 array, got {w.dtype} {tuple(w.shape)}")
    if bits not in (4, 8):
        raise ValueError(f"bits={bits}; this build covers 4 and 8")
    N, K = w.shape[0], w.shape[1] * 32 // bits
    if gs <= 0 or K % gs or tuple(s.shape) != (N, K // gs) or tuple(b.shape) != (N, K // gs):
        raise ValueError(f"scales {tuple(s.shape)} / biases {tuple(b.shape)} do not match "
                         f"w {tuple(w.shape)} at {bits} bits, group {gs}")
    if s.dtype != b.dtype:
        raise ValueError("scales and biases must share a dtype")
    return N, K


def _act_dtype(x: torch.Tensor, s: torch.Tensor) -> int:
    if x.dtype != s.dtype:
        raise ValueError(f"x is {x.dtype} but scales are {s.dtype}")
    return _dt(x)


# ----------------------------------------------------------------------------
# bindings: f(inputs, outputs, params) -> None


def b_dequant(ins, outs, p):
    w, s, b = ins
    (out,) = outs
    _require_gpu(w)
    _contig(w, s, b, out)
    gs, bits = int(p.get("group_size", 64)), int(p.get("bits", 4))
    N, K = _quant(w, s, b, bits, gs)
    if tuple(out.shape) != (N, K) or out.dtype != s.dtype:
        raise ValueError(f"dequant output must be {s.dtype} {(N, K)}")
    _check(lib().mi_affine_dequant(_ptr(w), _ptr(s), _ptr(b), _ptr(out), N, K, gs, bits, _dt(s),
                                   _stream(w)), "affine dequant")


def b_gather_dequant(ins, outs, p):
    ids, w, s, b = ins
    (out,) = outs
    _require_gpu(w)
    _contig(ids, w, s, b, out)
    gs, bits = int(p.get("group_size", 64)), int(p.get("bits", 4))
    N, K = _quant(w, s, b, bits, gs)
    if ids.dtype not in (torch.int32, torch.int64):
        raise ValueError("ids must be int32 or int64")
    n = ids.numel()
    if out.numel() != n * K or out.shape[-1] != K or out.dtype != s.dtype:
        raise ValueError(f"embedding output must be {s.dtype} [..., {K}] with {n} rows")
    _check(lib().mi_affine_gather_dequant(_ptr(ids), n, int(ids.dtype == torch.int64), _ptr(w),
                                          _ptr(s), _ptr(b), _ptr(out), N, K, gs, bits, _dt(s),
                                          _stream(w)), "quantized embedding")


def _qmm_dims(x, w, s, b, p):
    gs, bits = int(p.get("group_size", 64)), int(p.get("bits", 4))
    N, K = _quant(w, s, b, bits, gs)
    if x.shape[-1] != K:
        raise ValueError(f"x inner dim {x.shape[-1]} != K={K}")
    M = x.numel() // K if K else 0
    return M, N, K, gs, bits


def _out_like(y, x, N, name="output"):
    if y.dtype != x.dtype or tuple(y.shape) != (*x.shape[:-1], N):
        raise ValueError(f"{name} must be {x.dtype} {(*x.shape[:-1], N)}, got {y.dtype} {tuple(y.shape)}")


def _qmm_workspace(x, M, N, K, gs, bits, dt):
    """The K-part workspace of the _ws entries at this shape, or None (one
    K part: the plain entry)."""
    nbytes = int(lib().mi_qmm_workspace_bytes(M, N, K, gs, bits, dt))
    if nbytes == 0:
        return None
    return _workspace("qmm", x.device, _stream(x), nbytes, 8 << 20)


def b_qmm(ins, outs, p):
    x, w, s, b = ins
    (y,) = outs
    _require_gpu(x)
    _contig(x, w, s, b, y)
    M, N, K, gs, bits = _qmm_dims(x, w, s, b, p)
    dt = _act_dtype(x, s)
    _out_like(y, x, N)
    ws = _qmm_workspace(x, M, N, K, gs, bits, dt)
    if ws is not None:
        _check(lib().mi_qmm_affine_ws(_ptr(x), _ptr(w), _ptr(s), _ptr(b), _ptr(y), M, N, K, gs,
                                      bits, dt, _ptr(ws), ws.numel(), _stream(x)),
               "quantized matmul")
        return
    _check(lib().mi_qmm_affine(_ptr(x), _ptr(w), _ptr(s), _ptr(b), _ptr(y), M, N, K, gs, bits, dt,
                               _stream(x)), "quantized matmul")


def b_qmm_residual(ins, outs, p):
    x, w, s, b, r = ins
    (y,) = outs
    _require_gpu(x)
    _contig(x, w, s, b, r, y)
    M, N, K, gs, bits = _qmm_dims(x, w, s, b, p)
    dt = _act_dtype(x, s)
    _out_like(y, x, N)
    _out_like(r, x, N, "residual")
    ws = _qmm_workspace(x, M, N, K, gs, bits, dt)
    if ws is not None:
        _check(lib().mi_qmm_affine_residual_ws(_ptr(x), _ptr(w), _ptr(s), _ptr(b), _ptr(r),
                                               _ptr(y), M, N, K, gs, bits, dt, _ptr(ws),
                                               ws.numel(), _stream(x)), "qmm + residual")
        return
    _check(lib().mi_qmm_affine_residual(_ptr(x), _ptr(w), _ptr(s), _ptr(b), _ptr(r), _ptr(y), M,
                                        N, K, gs, bits, dt, _stream(x)), "qmm + residual")


def b_qmm_residual_rmsnorm(ins, outs, p):
    x, w, s, b, r, nw = ins
    h, y = outs
    _require_gpu(x)
    _contig(x, w, s, b, r, nw, h, y)
    M, N, K, gs, bits = _qmm_dims(x, w, s, b, p)
    dt = _act_dtype(x, s)
    for t, name in ((h, "h"), (y, "norm output"), (r, "residual")):
        _out_like(t, x, N, name)
    if tuple(nw.shape) != (N,) or nw.dtype != x.dtype:
        raise ValueError(f"norm weight must be {x.dtype} [{N}]")
    ws = _qmm_workspace(x, M, N, K, gs, bits, dt)
    if ws is not None:
        _check(lib().mi_qmm_affine_residual_rmsnorm_ws(
            _ptr(x), _ptr(w), _ptr(s), _ptr(b), _ptr(r), _ptr(nw), float(p["eps"]), _ptr(h),
            _ptr(y), M, N, K, gs, bits, dt, _ptr(ws), ws.numel(), _stream(x)),
            "qmm + residual + rms_norm")
        return
    _check(lib().mi_qmm_affine_residual_rmsnorm(_ptr(x), _ptr(w), _ptr(s), _ptr(b), _ptr(r),
                                                _ptr(nw), float(p["eps"]), _ptr(h), _ptr(y), M,
                                                N, K, gs, bits, dt, _stream(x)),
           "qmm + residual + rms_norm")


def b_qmm_split_gate(ins, outs, p):
    x, w, s, b = ins
    c, bx = outs
    _require_gpu(x)
    _contig(x, w, s, b, c, bx)
    M, N3, K, gs, bits = _qmm_dims(x, w, s, b, p)
    dt = _act_dtype(x, s)
    if N3 % 3:
        raise ValueError(f"split(3) needs N divisible by 3, got {N3}")
    _out_like(c, x, N3 // 3, "C")
    _out_like(bx, x, N3 // 3, "B*x")
    _check(lib().mi_qmm_affine_split_gate(_ptr(x), _ptr(w), _ptr(s), _ptr(b), _ptr(c), _ptr(bx),
                                          M, N3, K, gs, bits, dt, _stream(x)),
           "qmm + split + gate")


def b_qmm_dual(ins, outs, p):
    x, w1, s1, b1, w2, s2, b2 = ins
    act = int(p.get("act", MI_ACT_NONE))
    _require_gpu(x)
    _contig(x, w1, s1, b1, w2, s2, b2, *outs)
    M, N, K, gs, bits = _qmm_dims(x, w1, s1, b1, p)
    if _quant(w2, s2, b2, bits, gs) != (N, K):
        raise ValueError("the two weights of a dual qmm must have one shape")
    dt = _act_dtype(x, s1)
    if act == MI_ACT_SWIGLU:
        (y1,) = outs
        y2 = None
    else:
        y1, y2 = outs
        _out_like(y2, x, N)
    _out_like(y1, x, N)
    _check(lib().mi_qmm_affine_dual(_ptr(x), _ptr(w1), _ptr(s1), _ptr(b1), _ptr(w2), _ptr(s2),
                                    _ptr(b2), _ptr(y1), _ptr(y2), M, N, K, gs, bits, act, dt,
                                    _stream(x)), "dual qmm")


def b_qmm_grouped3(ins, outs, p):
    """ins: x, then (w, scales, biases) of each of the 3 projections; outs: 3."""
    if len(ins) != 10 or len(outs) != 3:
        raise ValueError("grouped qmm takes x + 3 x (w, scales, biases) and gives 3 outputs")
    x = ins[0]
    parts = [ins[1 + 3 * i: 4 + 3 * i] for i in range(3)]
    _require_gpu(x)
    _contig(x, *ins[1:], *outs)
    Ns = []
    for (w, s, b), y in zip(parts, outs):
        M, N, K, gs, bits = _qmm_dims(x, w, s, b, p)
        _out_like(y, x, N)
        Ns.append(N)
    dt = _act_dtype(x, parts[0][1])
    ptrs = (ctypes.c_void_p * 3)
    _check(lib().mi_qmm_affine_grouped3(
        _ptr(x), ptrs(*[_ptr(w) for w, _, _ in parts]), ptrs(*[_ptr(s) for _, s, _ in parts]),
        ptrs(*[_ptr(b) for _, _, b in parts]), ptrs(*[_ptr(y) for y in outs]), M,
        (ctypes.c_int64 * 3)(*Ns), K, gs, bits, dt, _stream(x)), "grouped qmm")


def b_rms_norm(ins, outs, p):
    x, w = ins
    (y,) = outs
    _require_gpu(x)
    _contig(x, w, y)
    D = x.shape[-1]
    if tuple(w.shape) != (D,) or w.dtype != x.dtype or y.shape != x.shape or y.dtype != x.dtype:
        raise ValueError("rms_norm: weight must be [D] and the output like x, in x's dtype")
    _check(lib().mi_rms_norm(_ptr(x), _ptr(w), _ptr(y), x.numel() // D if D else 0, D,
                             float(p["eps"]), _dt(x), _stream(x)), "rms_norm")


def b_norm_rope(ins, outs, p):
    """x [B, L, H*D] (or w absent: rope only) -> out [B, H, L, D]."""
    x = ins[0]
    w = ins[1] if len(ins) > 1 else None
    (out,) = outs
    _require_gpu(x)
    _contig(x, w, out)
    H = int(p["n_heads"])
    B, L, HD = x.shape
    if HD % H:
        raise ValueError(f"last dim {HD} is not divisible by {H} heads")
    D = HD // H
    if tuple(out.shape) != (B, H, L, D) or out.dtype != x.dtype:
        raise ValueError(f"norm_rope output must be {x.dtype} {(B, H, L, D)}")
    if w is not None and (tuple(w.shape) != (D,) or w.dtype != x.dtype):
        raise ValueError(f"norm weight must be {x.dtype} [{D}]")
    _check(lib().mi_norm_rope(_ptr(x), _ptr(w), _ptr(out), B, L, H, D, HD,
                              float(p.get("eps", 0.0)), int(p.get("dims", D)),
                              int(p.get("traditional", 0)), float(p.get("base", 10000.0)),
                              float(p.get("scale", 1.0)), int(p.get("offset", 0)), L, 0, _dt(x),
                              _stream(x)), "norm_rope")


def b_sdpa(ins, outs, p):
    q, k, v = ins
    (o,) = outs
    _require_gpu(q)
    _contig(q, k, v, o)
    B, H, Lq, D = q.shape
    _, HK, Lk, _ = k.shape
    if tuple(v.shape) != tuple(k.shape) or k.shape[0] != B or k.shape[3] != D:
        raise ValueError(f"sdpa shapes q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)}")
    layout = int(p.get("out_layout", 0))
    want = (B, H, Lq, D) if layout == 0 else (B, Lq, H, D)
    if tuple(o.shape) != want or o.dtype != q.dtype or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"sdpa output must be {q.dtype} {want}")
    _check(lib().mi_sdpa(_ptr(q), _ptr(k), _ptr(v), _ptr(o), B, H, HK, Lq, Lk, D, Lk,
                         float(p["scale"]), int(p.get("causal", 1)), layout, _dt(q), _stream(q)),
           "sdpa")


def b_swiglu(ins, outs, p):
    g, u = ins
    (y,) = outs
    _require_gpu(g)
    _contig(g, u, y)
    if g.shape != u.shape or y.shape != g.shape or not (g.dtype == u.dtype == y.dtype):
        raise ValueError("swiglu operands must share shape and dtype")
    _check(lib().mi_swiglu(_ptr(g), _ptr(u), _ptr(y), g.numel(), _dt(g), _stream(g)), "swiglu")


def b_shortconv(ins, outs, p):
    bx, c, w = ins[:3]
    state = ins[3] if len(ins) > 3 else None
    out, state_out = outs
    _require_gpu(bx)
    _contig(bx, c, w, state, out, state_out)
    B, L, D = bx.shape
    if c.shape != bx.shape or out.shape != bx.shape or tuple(state_out.shape) != (B, 2, D):
        raise ValueError("shortconv shapes")
    if w.numel() != 3 * D or (state is not None and tuple(state.shape) != (B, 2, D)):
        raise ValueError("shortconv weight must hold [D, 3] values and the state [B, 2, D]")
    _check(lib().mi_shortconv(_ptr(bx), _ptr(c), _ptr(w), _ptr(state), _ptr(out),
                              _ptr(state_out), B, L, D, _dt(bx), _stream(bx)), "shortconv")


def b_linear_f32(ins, outs, p):
    x, w = ins[:2]
    bias = ins[2] if len(ins) > 2 else None
    (y,) = outs
    _require_gpu(x)
    _contig(x, w, bias, y)
    if any(t is not None and t.dtype != torch.float32 for t in (x, w, bias, y)):
        raise ValueError("linear_f32 takes float32 arrays")
    K = x.shape[-1]
    N = w.shape[0]
    if w.shape[1] != K or (bias is not None and tuple(bias.shape) != (N,)):
        raise ValueError("linear_f32 shapes")
    _out_like(y, x, N)
    _check(lib().mi_linear_f32(_ptr(x), _ptr(w), _ptr(bias), _ptr(y), x.numel() // K, N, K,
                               int(p.get("act", MI_ACT_NONE)), _stream(x)), "linear_f32")


# Workspaces (the K-part sums of the _ws qmm entries, mi_gelu_mlp_f32's
# tickets and partial sums), zero-filled when made; mi_gelu_mlp_f32 leaves its
# tickets zero after every call.
#
# Eager calls share one workspace per (kind, device, stream): calls on one
# stream run in order. A call under HIP graph capture bakes the workspace's
# address into the graph, and graphs may later replay on different streams at
# the same time, so a captured call never takes an eager stream's workspace:
# inside graph_workspaces() every graph captured in the scope shares the
# scope's own workspaces (its calls are stream-ordered), and a capture outside
# such a scope gives each call a workspace of its own. Either way the buffer is
# kept alive as long as the process, since a graph may replay at any time; a
# workspace that has to grow is replaced and the old one kept alive too.
_workspaces: dict[tuple, torch.Tensor] = {}
_retired: list[torch.Tensor] = []
_scope = threading.local()


@contextlib.contextmanager
def graph_workspaces():
    """A scope whose graph captures share workspaces of their own (no other
    graph or stream uses them). GraphWrapper captures each graph in one."""
    prev = getattr(_scope, "token", None)
    _scope.token = object()
    try:
        yield
    finally:
        _scope.token = prev


def _workspace(kind: str, device, stream: int, nbytes: int, minimum: int = 4096) -> torch.Tensor:
    size = max(nbytes, minimum)
    if torch.cuda.is_current_stream_capturing():
        token = getattr(_scope, "token", None)
        if token is None:  # a capture of its own: a workspace per call
            ws = torch.zeros(size, dtype=torch.uint8, device=device)
            _retired.append(ws)
            return ws
        key = (kind, device, token)
    else:
        key = (kind, device, stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _retired.append(ws)
        ws = torch.zeros(size, dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


def b_gelu_mlp_f32(ins, outs, p):
    """inputs (x [M, K], w1 [H, K], b1 [H], w2 [N, H], b2 [N]) -> y [M, N]."""
    x, w1, b1, w2, b2 = ins
    (y,) = outs
    _require_gpu(x)
    _contig(x, w1, b1, w2, b2, y)
    if any(t.dtype != torch.float32 for t in (x, w1, b1, w2, b2, y)):
        raise ValueError("gelu_mlp_f32 takes float32 arrays")
    if x.dim() != 2 or w1.dim() != 2 or w2.dim() != 2:
        raise ValueError("gelu_mlp_f32 takes 2-d x, w1, w2")
    M, K = x.shape
    H, N = w1.shape[0], w2.shape[0]
    if (w1.shape[1] != K or w2.shape[1] != H or tuple(b1.shape) != (H,)
            or tuple(b2.shape) != (N,) or tuple(y.shape) != (M, N)):
        raise ValueError("gelu_mlp_f32 shapes")
    stream = _stream(x)
    nbytes = int(lib().mi_gelu_mlp_f32_workspace_bytes(M, K, H, N))
    ws = _workspace("gelu_mlp", x.device, stream, nbytes)
    _check(lib().mi_gelu_mlp_f32(_ptr(x), _ptr(w1), _ptr(b1), _ptr(w2), _ptr(b2), _ptr(y), M, K,
                                 H, N, _ptr(ws), ws.numel(), stream), "gelu_mlp_f32")


def b_argmax(ins, outs, p):
    (x,) = ins
    (o,) = outs
    _require_gpu(x)
    _contig(x, o)
    V = x.shape[-1]
    if o.dtype != torch.int32 or o.numel() != x.numel() // V:
        raise ValueError("argmax output must be int32 with one entry per row")
    rows = x.numel() // V
    # split path: a workspace from torch's allocator (graph-capture safe); the
    # one-workgroup path (no workspace) when p["split"] is False
    ws, nbytes = None, 0
    if p.get("split", True) and 0 < rows <= 65535:
        nbytes = int(lib().mi_argmax_workspace_bytes(rows, V))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    _check(lib().mi_argmax(_ptr(x), _ptr(o), rows, V, _dt(x), _ptr(ws), nbytes, _stream(x)),
           "argmax")


BINDINGS: dict[str, Callable] = {
    "mi_affine_dequant": b_dequant,
    "mi_affine_gather_dequant": b_gather_dequant,
    "mi_qmm_affine": b_qmm,
    "mi_qmm_affine_residual": b_qmm_residual,
    "mi_qmm_affine_residual_rmsnorm": b_qmm_residual_rmsnorm,
    "mi_qmm_affine_split_gate": b_qmm_split_gate,
    "mi_qmm_affine_dual": b_qmm_dual,
    "mi_qmm_affine_grouped3": b_qmm_grouped3,
    "mi_rms_norm": b_rms_norm,
    "mi_norm_rope": b_norm_rope,
    "mi_sdpa": b_sdpa,
    "mi_swiglu": b_swiglu,
    "mi_shortconv": b_shortconv,
    "mi_linear_f32": b_linear_f32,
    "mi_gelu_mlp_f32": b_gelu_mlp_f32,
    "mi_argmax": b_argmax,
}


def binding(symbol: str) -> Callable:
    """The binding of a C-ABI entry point named by a KernelSpec's ``source``.
    An unknown name is a build error (RuntimeError), as a Metal body that does
    not compile is in the reference (ladder/child.py:43)."""
    fn = BINDINGS.get(symbol)
    if fn is None:
        raise RuntimeError(f"Unable to bind kernel source {symbol!r}: not an entry point of "
                           f"{LIB_PATH.name} (known: {sorted(BINDINGS)})")
    return fn
