"""GPU parity of the fused q/k/v projections + attention prologue
(mi_qmm_affine_qkv_norm_rope, ops.qkv_norm_rope) through the C ABI.

Bar: bit for bit equal to the two entries it replaces (mi_qmm_affine_grouped3,
then mi_norm_rope_qkv), whose own parity with the oracle the kernel tests hold;
and within the bf16/fp16 region tolerance (1e-2 max-abs-normalised) of the
oracle's quantized_matmul followed by its norm_rope. Shapes: the Qwen3 layer
(32 q heads, 8 kv heads, D 128, K 2560) at the prefill sizes and the LFM2
attention layer (D 64, K 2048) at 2048 tokens, 4- and 8-bit weights, ragged
token counts, two sequences, a cache offset, and the shapes the fused entry
declines.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import packed_to_torch, rng, to_torch

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from autotuner_runtime import numeric, ops  # noqa: E402

EPS, BASE = 1e-6, 1e6


def _case(seed, B, L, H, HK, D, K, dtype, bits=4):
    r = rng(seed)
    x = oracle.round_to(r.normal(0, 1, (B, L, K)), dtype)
    qs = [oracle.quantize_affine(r.normal(0, 0.02, (n, K)).astype(np.float32), 64, bits, dtype)
          for n in (H * D, HK * D, HK * D)]
    qn = oracle.round_to(1 + 0.2 * r.normal(0, 1, D), dtype)
    kn = oracle.round_to(1 + 0.2 * r.normal(0, 1, D), dtype)
    ws = [(packed_to_torch(w), to_torch(s, dtype), to_torch(b, dtype)) for w, s, b in qs]
    return x, qs, qn, kn, ws


def _caches(B, HK, cap, D, tdt):
    kc = torch.full((B, HK, cap, D), 5.0, dtype=tdt, device="cuda")
    return kc, torch.full_like(kc, 6.0)


@pytest.mark.parametrize("B,L,offset,K,dtype,D,bits", [
    (1, 128, 0, 2560, "bfloat16", 128, 4),   # the Qwen3 prefill step
    (1, 100, 0, 2560, "bfloat16", 128, 4),   # ragged last token tile
    (1, 9, 17, 512, "bfloat16", 128, 4),     # smallest MFMA-path size, cache offset
    (2, 40, 3, 512, "bfloat16", 128, 4),     # two sequences: positions restart per sequence
    (1, 256, 0, 512, "float16", 128, 4),     # the largest size the fused form takes at D 128
    (1, 128, 5, 512, "bfloat16", 128, 8),
    (1, 2048, 0, 2048, "bfloat16", 64, 4),   # the LFM2 prefill's attention layers
    (1, 520, 40, 512, "bfloat16", 64, 8),    # ragged, cache offset
    (2, 300, 0, 512, "float16", 64, 4),
])
def test_qkv_norm_rope_equals_two_entries(B, L, offset, K, dtype, D, bits):
    H, HK, cap = 32, 8, offset + L + 5
    tdt = torch.bfloat16 if dtype == "bfloat16" else torch.float16
    x, qs, qn, kn, ws = _case(1200 + L + B + offset + D + bits, B, L, H, HK, D, K, dtype, bits)
    xd, qw, kw = to_torch(x, dtype), to_torch(qn, dtype), to_torch(kn, dtype)
    kc, vc = _caches(B, HK, cap, D, tdt)
    got = ops.qkv_norm_rope(xd, ws, qw, kw, H, HK, EPS, D, BASE, offset, kc, vc, offset, 64, bits)
    assert got is not None, "the fused entry should cover this shape"
    kc2, vc2 = _caches(B, HK, cap, D, tdt)
    q, k, v = ops.qmm_grouped3(xd, ws, 64, bits)
    want = ops.norm_rope_qkv(q, k, v, qw, kw, H, HK, EPS, D, BASE, offset, kc2, vc2, offset)
    assert torch.equal(got, want)
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
    # rows outside [offset, offset + L) untouched
    assert bool((kc[:, :, :offset] == 5.0).all()) and bool((vc[:, :, offset + L:] == 6.0).all())
    # against the oracle (first sequence; q heads 0 and 31, the k cache rows)
    x0 = x[:1, :128]
    yq = oracle.quantized_matmul(x0, *qs[0], 64, bits, dtype)
    yk = oracle.quantized_matmul(x0, *qs[1], 64, bits, dtype)
    wq = oracle.norm_rope(yq, qn, EPS, H, D, BASE, offset, dtype)
    wk = oracle.norm_rope(yk, kn, EPS, HK, D, BASE, offset, dtype)
    for got_t, want_t in ((got[:1, [0, H - 1], :128], wq[:, [0, H - 1]]),
                          (kc[:1, :, offset:offset + min(L, 128)], wk)):
        t = numeric.max_abs_normalised(got_t.cpu(), to_torch(want_t, dtype, "cpu"))
        assert t.passed, f"max-abs-normalised error {t.error:.3e} > {t.tol:.1e} ({t.detail})"


def test_qkv_norm_rope_replays_in_a_graph():
    """Captured in a HIP graph (the bench's form): every replay, with eager work
    between replays, equals the eager call."""
    B, L, H, HK, D, K = 1, 128, 32, 8, 128, 512
    x, _, qn, kn, ws = _case(1290, B, L, H, HK, D, K, "bfloat16")
    xd, qw, kw = to_torch(x, "bfloat16"), to_torch(qn, "bfloat16"), to_torch(kn, "bfloat16")
    kc, vc = _caches(B, HK, L, D, torch.bfloat16)
    want = ops.qkv_norm_rope(xd, ws, qw, kw, H, HK, EPS, D, BASE, 0, kc, vc, 0)
    kw_, vw_ = kc.clone(), vc.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.qkv_norm_rope(xd, ws, qw, kw, H, HK, EPS, D, BASE, 0, kc, vc, 0)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = ops.qkv_norm_rope(xd, ws, qw, kw, H, HK, EPS, D, BASE, 0, kc, vc, 0)
    for _ in range(3):
        kc.fill_(0.0)
        vc.fill_(0.0)
        out.fill_(0.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want) and torch.equal(kc, kw_) and torch.equal(vc, vw_)


@pytest.mark.parametrize("what", ["head64", "head96", "fp32", "decode", "long", "traditional",
                                  "no_norm"])
def test_qkv_norm_rope_declines_uncovered_shapes(what):
    """Shapes outside the fused form return None and launch nothing: the caller
    then runs grouped3 + norm_rope_qkv (the Qwen3 region model does)."""
    B, L, H, HK, D, K = 1, 16, 8, 2, 128, 256
    dtype, bits, trad = "bfloat16", 4, False
    if what == "head64":  # 64-value heads below 512 tokens
        D = 64
    elif what == "head96":
        D = 96
    elif what == "fp32":
        dtype = "float32"
    elif what == "decode":
        L = 4
    elif what == "long":  # 128-value heads past 256 tokens: the two launches are faster
        L = 264
    elif what == "traditional":
        trad = True
    x, _, qn, kn, ws = _case(1300, B, L, H, HK, D, K, dtype, bits)
    tdt = {"bfloat16": torch.bfloat16, "float32": torch.float32}[dtype]
    kc, vc = _caches(B, HK, L, D, tdt)
    qw = to_torch(qn, dtype)
    kw = None if what == "no_norm" else to_torch(kn, dtype)
    if kw is None:  # a missing norm weight is declined by the C entry (null pointer)
        from autotuner_runtime import hip
        import ctypes
        ptrs = ctypes.c_void_p * 3
        out = torch.empty((B, H, L, D), dtype=tdt, device="cuda")
        st = hip.lib().mi_qmm_affine_qkv_norm_rope(
            to_torch(x, dtype).data_ptr(), ptrs(*[w.data_ptr() for w, _, _ in ws]),
            ptrs(*[s.data_ptr() for _, s, _ in ws]), ptrs(*[b.data_ptr() for _, _, b in ws]),
            qw.data_ptr(), None, out.data_ptr(), kc.data_ptr(), vc.data_ptr(), B, L, H, HK, D, K,
            64, bits, EPS, D, 0, BASE, 1.0, 0, L, 0, hip._dt(out),
            torch.cuda.current_stream().cuda_stream)
        assert st == hip.MI_ERR_UNSUPPORTED
    else:
        got = ops.qkv_norm_rope(to_torch(x, dtype), ws, qw, kw, H, HK, EPS, D, BASE, 0, kc, vc, 0,
                                64, bits, traditional=trad)
        assert got is None
    torch.cuda.synchronize()
    assert bool((kc == 5.0).all()) and bool((vc == 6.0).all())


def test_qkv_norm_rope_rejects_a_short_cache():
    B, L, H, HK, D, K = 1, 16, 8, 2, 128, 256
    x, _, qn, kn, ws = _case(1310, B, L, H, HK, D, K, "bfloat16")
    kc, vc = _caches(B, HK, L, D, torch.bfloat16)
    with pytest.raises(ValueError, match="capacity"):
        ops.qkv_norm_rope(to_torch(x, "bfloat16"), ws, to_torch(qn, "bfloat16"),
                          to_torch(kn, "bfloat16"), H, HK, EPS, D, BASE, 4, kc, vc, 4)
