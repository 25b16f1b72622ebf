"""GPU parity of every HIP kernel against the CPU oracle, through the C ABI.

Bars: bit-exact for dequant, integer/index outputs and the one-hot cases;
otherwise the port's region criterion max|c - r| <= tol * max|r| with
tol 1e-2 for bf16/fp16 and 1e-5 for fp32 (numeric.max_abs_normalised).
Shapes are the benchmark's config 2 (x[M, 2560] @ W[9728, 2560]^T, M in 1/16/128),
the Qwen3/LFM2 projection shapes, and ragged edges.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
from conftest import packed_to_torch, rng, to_np, to_torch

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from autotuner_runtime import hip, numeric, ops  # noqa: E402


def _close(got, want, dtype, tol=None):
    t = numeric.max_abs_normalised(to_torch(got, dtype, "cpu") if isinstance(got, np.ndarray) else got.cpu(),
                                   to_torch(want, dtype, "cpu"), tol)
    assert t.passed, f"max-abs-normalised error {t.error:.3e} > {t.tol:.1e} ({t.detail})"
    return t.error


def _quant(seed, N, K, gs=64, bits=4, dtype="bfloat16"):
    r = rng(seed)
    return oracle.quantize_affine(r.normal(0, 0.02, (N, K)).astype(np.float32), gs, bits, dtype)


def _dev(wq, s, b, dtype):
    return packed_to_torch(wq), to_torch(s, dtype), to_torch(b, dtype)


# ---------------------------------------------------------------------- A1


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("bits,gs", [(4, 64), (4, 32), (4, 128), (8, 64), (8, 128)])
def test_dequant_bit_exact(dtype, bits, gs):
    wq, s, b = _quant(100 + bits + gs, 96, 1024, gs, bits, dtype)
    want = oracle.dequantize(wq, s, b, gs, bits, dtype)
    got = ops.dequantize(*_dev(wq, s, b, dtype), group_size=gs, bits=bits)
    assert np.array_equal(to_np(got).view(np.uint32), want.view(np.uint32))


def test_dequant_config2_shape_bit_exact():
    wq, s, b = _quant(7, 9728, 2560)
    want = oracle.dequantize(wq, s, b, 64, 4, "bfloat16")
    got = ops.dequantize(*_dev(wq, s, b, "bfloat16"))
    assert np.array_equal(to_np(got).view(np.uint32), want.view(np.uint32))


def _onehot_x(M, K, seed):
    """x rows holding a single 1.0, at column cols[m]: x @ W^T then reads
    column cols[m] of the dequantized W exactly (one nonzero product, fp32
    accumulation, a bf16 store of a bf16 value)."""
    cols = rng(seed).integers(0, K, M)
    x = np.zeros((1, M, K), np.float32)
    x[0, np.arange(M), cols] = 1.0
    return x, cols


@pytest.mark.parametrize("M", [16, 128])
@pytest.mark.parametrize("case", ["quantized", "tiny_bias", "edges"])
def test_qmm_mfma_dequant_bit_exact_one_hot(M, case):
    """A1 inside the MFMA GEMM, bit for bit: with one-hot x rows, y[m, n] is
    W[n, cols[m]] of the dequantized matrix, so every dequantized value the
    MFMAs consumed is checked against the oracle. 'quantized' groups come from
    the affine quantizer; 'tiny_bias' groups have b = ±s/1024; 'edges' mixes
    zero scales, zero biases, negative scales and b/s exponent gaps from 2^-6
    to 2^22. M = 16 runs 32-token tiles, M = 128 64-token tiles; the dual
    output runs the register-prefetched two-part tile."""
    N, K = 2048, 2560
    wq, s, b = _quant(780, N, K)
    r = rng(781)
    if case == "tiny_bias":
        b = oracle.round_to(s * np.float32(2.0 ** -10) * r.choice([-1, 1], s.shape), "bfloat16")
    elif case == "edges":
        pick = r.integers(0, 6, s.shape)
        gap = np.float32(2.0) ** r.integers(-6, 23, s.shape).astype(np.float32)
        b_gap = oracle.round_to(np.abs(s) * gap * r.choice([-1, 1], s.shape), "bfloat16")
        s = np.where(pick == 0, 0.0, np.where(pick == 1, -s, s)).astype(np.float32)
        b = np.where(pick == 2, 0.0, np.where(pick >= 3, b_gap, b)).astype(np.float32)
    want = oracle.dequantize(wq, s, b, 64, 4, "bfloat16")
    x, cols = _onehot_x(M, K, 782 + M)
    xd = to_torch(x, "bfloat16")
    w = _dev(wq, s, b, "bfloat16")
    expect = np.ascontiguousarray(want[:, cols].T)
    got = to_np(ops.quantized_matmul(xd, *w))[0]
    assert np.array_equal(got.view(np.uint32), expect.view(np.uint32))
    for part in ops.qmm_dual(xd, *w, *w):
        assert np.array_equal(to_np(part)[0].view(np.uint32), expect.view(np.uint32))


def test_quantized_embedding_gathers_dequantized_rows():
    wq, s, b = _quant(8, 500, 256)
    W = oracle.dequantize(wq, s, b, 64, 4, "bfloat16")
    ids = np.array([[3, 0, 499, 3, 17]], np.int64)
    for idt in (torch.int64, torch.int32):
        got = ops.quantized_embedding(torch.from_numpy(ids).to("cuda", idt), *_dev(wq, s, b, "bfloat16"))
        assert got.shape == (1, 5, 256)
        assert np.array_equal(to_np(got)[0], W[ids[0]])


# ------------------------------------------------------------------- A2-A4


@pytest.mark.parametrize("M", [1, 2, 5, 8, 9, 16, 33, 64, 100, 128, 300])
def test_qmm_config2_shape(M):
    """Config 2 shapes (M in 1/16/128) and the GEMV/MFMA switch
    points around them."""
    r = rng(200 + M)
    K, N = 2560, 9728
    x = oracle.round_to(r.normal(0, 1, (M, K)), "bfloat16")
    wq, s, b = _quant(7, N, K)
    y = ops.quantized_matmul(to_torch(x, "bfloat16"), *_dev(wq, s, b, "bfloat16"))
    if M <= 16:
        want = oracle.qmm_factored(x, wq, s, b, 64, 4, "bfloat16")
    else:
        want = oracle.quantized_matmul(x, wq, s, b, 64, 4, "bfloat16")
    _close(y, want, "bfloat16")


@pytest.mark.parametrize("M,N", [(2, 9728), (3, 9728), (4, 9004), (1, 9004)])
@pytest.mark.parametrize("resid", [False, True])
def test_qmv_wide_workgroups_equal_four_wave_ones(M, N, resid):
    """The decode GEMV sizes its workgroups from N and the CU count (up to 16
    waves, so the rows spread evenly over the CUs). A row's arithmetic does
    not depend on the workgroup: the first 2048 rows of the wide launch equal,
    bit for bit, a launch over those rows alone (4 waves). N = 9004 leaves a
    partial last workgroup; M = 3 leaves a token of the 4-token blocks empty;
    M = 1 at K = 5120 runs without the early weight prefetch, a row a wave.
    Both against qmm_factored at the bf16 bar."""
    r = rng(260 + M + N)
    K = 5120 if M == 1 else 2560
    x = oracle.round_to(r.normal(0, 1, (M, K)), "bfloat16")
    wq, s, b = _quant(17, N, K)
    res = oracle.round_to(r.normal(0, 1, (M, N)), "bfloat16")
    dev = _dev(wq, s, b, "bfloat16")
    xd, rd = to_torch(x, "bfloat16"), to_torch(res, "bfloat16")
    head = [t[:2048].contiguous() for t in dev]
    if resid:
        wide = ops.qmm_residual(xd, *dev, rd)
        narrow = ops.qmm_residual(xd, *head, rd[:, :2048].contiguous())
    else:
        wide = ops.quantized_matmul(xd, *dev)
        narrow = ops.quantized_matmul(xd, *head)
    assert torch.equal(wide[:, :2048], narrow)
    t = oracle.qmm_factored(x, wq, s, b, 64, 4, "bfloat16")
    want = oracle.round_to(res.astype(np.float64) + t, "bfloat16") if resid else t
    _close(wide, want, "bfloat16")


@pytest.mark.parametrize("M,N,K", [(1, 2560, 9728), (2, 2048, 8192), (4, 600, 9728), (1, 8, 4160)])
def test_qmv_row_per_wave_long_k(M, N, K):
    """Past K = 4096 the single-output decode GEMV gives each row a whole wave
    (64 lanes; about 5 chunks a lane at K = 9728, the Qwen3 down_proj at
    decode) and adds its four 16-lane sums in a fixed order. Within the bf16
    bar of qmm_factored, with and without the residual; N = 8 is a grid of
    fewer rows than one workgroup holds."""
    r = rng(1500 + M + N + K)
    x = oracle.round_to(r.normal(0, 1, (M, K)), "bfloat16")
    res = oracle.round_to(r.normal(0, 1, (M, N)), "bfloat16")
    wq, s, b = _quant(1501, N, K)
    dev = _dev(wq, s, b, "bfloat16")
    xd, rd = to_torch(x, "bfloat16"), to_torch(res, "bfloat16")
    t = oracle.qmm_factored(x, wq, s, b, 64, 4, "bfloat16")
    _close(ops.quantized_matmul(xd, *dev), t, "bfloat16")
    _close(ops.qmm_residual(xd, *dev, rd), oracle.round_to(res.astype(np.float64) + t, "bfloat16"),
           "bfloat16")


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("bits,gs", [(4, 64), (8, 64), (4, 32), (4, 128), (8, 32)])
@pytest.mark.parametrize("M", [1, 7, 40, 130, 520])
def test_qmm_dtypes_bits_groups(dtype, bits, gs, M):
    r = rng(300 + M + bits)
    K, N = 512, 200  # N not a multiple of 32: ragged output tiles
    x = oracle.round_to(r.normal(0, 1, (M, K)), dtype)
    wq, s, b = _quant(9 + bits, N, K, gs, bits, dtype)
    y = ops.quantized_matmul(to_torch(x, dtype), *_dev(wq, s, b, dtype), group_size=gs, bits=bits)
    if dtype == "float32":
        # fp32 runs the per-group factored sum at every M (the GEMV kernels;
        # the MFMA tiles take 16-bit T only): held to north_star's fp32 bar
        # against the oracle's restatement of that same algorithm
        # (scaffold/lower.py:1179-1233), and to twice it against the
        # dequantize-first form
        _close(y, oracle.qmm_factored(x, wq, s, b, gs, bits, dtype), dtype, 1e-5)
        _close(y, oracle.quantized_matmul(x, wq, s, b, gs, bits, dtype), dtype, 2e-5)
    else:
        _close(y, oracle.quantized_matmul(x, wq, s, b, gs, bits, dtype), dtype)


@pytest.mark.parametrize("M", [1, 64, 128])
def test_qmm_special_cases(M):
    """x = 0 -> 0 exactly; one-hot rows -> dequantized columns exactly."""
    K, N = 1024, 96
    wq, s, b = _quant(11, N, K)
    W = oracle.dequantize(wq, s, b, 64, 4, "bfloat16")
    dev = _dev(wq, s, b, "bfloat16")
    zero = ops.quantized_matmul(torch.zeros((M, K), dtype=torch.bfloat16, device="cuda"), *dev)
    assert bool((zero == 0).all())
    x = np.zeros((M, K), np.float32)
    ks = (np.arange(M) * 37) % K
    x[np.arange(M), ks] = 1.0
    y = to_np(ops.quantized_matmul(to_torch(x, "bfloat16"), *dev))
    assert np.array_equal(y, W[:, ks].T)


@pytest.mark.parametrize("M", [3, 70])
def test_qmm_k_off_the_mfma_step_uses_generic_path(M):
    """K = 160 at group 32: a valid MLX shape that is not a multiple of the
    MFMA kernel's 64-value super-step, so every M runs the generic kernel."""
    r = rng(12)
    x = oracle.round_to(r.normal(0, 1, (M, 160)), "bfloat16")
    wq, s, b = _quant(13, 64, 160, gs=32)
    y = ops.quantized_matmul(to_torch(x, "bfloat16"), *_dev(wq, s, b, "bfloat16"), group_size=32)
    _close(y, oracle.quantized_matmul(x, wq, s, b, 32, 4, "bfloat16"), "bfloat16")


def test_qmm_rejects_bad_shapes():
    wq, s, b = _quant(14, 32, 256)
    dev = _dev(wq, s, b, "bfloat16")
    with pytest.raises(ValueError):
        ops.quantized_matmul(torch.zeros((2, 128), dtype=torch.bfloat16, device="cuda"), *dev)
    with pytest.raises(ValueError):
        ops.quantized_matmul(torch.zeros((2, 256), dtype=torch.bfloat16, device="cuda"), *dev, bits=3)


# ---------------------------------------------------------- region epilogues


@pytest.mark.parametrize("M,N,bits", [(1, 512, 4), (16, 512, 4), (128, 512, 4), (520, 512, 4),
                                       (520, 510, 4), (520, 512, 8)])
def test_qmm_residual(M, N, bits):
    """[qmm, add]. M = 520 runs 128-token tiles (a last tile of 8 tokens)
    whose epilogue loads every residual of a wave before its first store;
    N = 510 (not a multiple of 4) takes the element-wise epilogue."""
    r = rng(400 + M + N + bits)
    K = 2048
    x = oracle.round_to(r.normal(0, 1, (1, M, K)), "bfloat16")
    res = oracle.round_to(r.normal(0, 1, (1, M, N)), "bfloat16")
    wq, s, b = _quant(15, N, K, bits=bits)
    y = ops.qmm_residual(to_torch(x, "bfloat16"), *_dev(wq, s, b, "bfloat16"), to_torch(res, "bfloat16"),
                         bits=bits)
    t = oracle.quantized_matmul(x, wq, s, b, 64, bits, "bfloat16")
    _close(y, oracle.round_to(res.astype(np.float64) + t, "bfloat16"), "bfloat16")


@pytest.mark.parametrize("M", [1, 128])
def test_qmm_residual_rmsnorm(M):
    r = rng(500 + M)
    K, N = 1024, 2048
    x = oracle.round_to(r.normal(0, 1, (1, M, K)), "bfloat16")
    res = oracle.round_to(r.normal(0, 1, (1, M, N)), "bfloat16")
    nw = oracle.round_to(1 + 0.1 * r.normal(0, 1, N), "bfloat16")
    wq, s, b = _quant(16, N, K)
    h, y = ops.qmm_residual_rmsnorm(to_torch(x, "bfloat16"), *_dev(wq, s, b, "bfloat16"),
                                    to_torch(res, "bfloat16"), to_torch(nw, "bfloat16"), 1e-5)
    h_want = oracle.round_to(res.astype(np.float64) + oracle.quantized_matmul(x, wq, s, b, 64, 4, "bfloat16"), "bfloat16")
    _close(h, h_want, "bfloat16")
    # the norm stage is checked on the kernel's own h: bit-level agreement of the
    # two-rounding form up to the rsqrt's last bit
    _close(y, oracle.rms_norm(to_np(h), nw, 1e-5, "bfloat16"), "bfloat16")


# ----------------------------------------------------------------- K parts


def _kparts_call(name, *args):
    st = torch.cuda.current_stream().cuda_stream
    status = getattr(hip.lib(), name)(*args, st)
    assert status == 0, hip.lib().mi_last_error()


@pytest.mark.parametrize("M,N,K,bits,dtype", [
    (128, 2560, 4096, 4, "bfloat16"),   # o_proj: 4 K parts of 4 stages
    (128, 2560, 9728, 4, "bfloat16"),   # down_proj: 4 parts of 9 or 10 stages
    (100, 200, 4096, 8, "bfloat16"),    # ragged M and N, 8-bit
    (40, 512, 8192, 4, "float16"),      # 64-token part tiles
    (72, 520, 4096, 4, "float16"),      # fp16 with 4 parts, ragged M
    (16, 256, 4224, 4, "bfloat16"),     # 66 stages, two waves a part: chunks of 8 / 9
])
def test_qmm_k_parts_workspace_equals_one_launch(M, N, K, bits, dtype):
    """At shapes with K parts the _ws entries (the parts as workgroups of their
    own, then a kernel that adds them) equal, bit for bit, the entries without
    a workspace (each workgroup runs the parts in turn), for [qmm], [qmm, add]
    and [qmm, add, rms_norm]; and both are within tolerance of the oracle. A
    workspace one byte short takes the one-launch path, same bits."""
    L = hip.lib()
    r = rng(900 + M + K)
    dt = hip._DT[getattr(torch, dtype)]
    x = oracle.round_to(r.normal(0, 1, (M, K)), dtype)
    res = oracle.round_to(r.normal(0, 1, (M, N)), dtype)
    nw = oracle.round_to(1 + 0.1 * r.normal(0, 1, N), dtype)
    q = _quant(901, N, K, 64, bits, dtype)
    xd, rd, nwd = to_torch(x, dtype), to_torch(res, dtype), to_torch(nw, dtype)
    w, s, b = _dev(*q, dtype)
    nbytes = L.mi_qmm_workspace_bytes(M, N, K, 64, bits, dt)
    assert nbytes == 4 * M * N * 4  # four K parts
    ws = torch.full((nbytes,), 0xFF, dtype=torch.uint8, device="cuda")  # NaN partials
    P = hip._ptr
    ys = {}
    for mode, (wsp, wsb) in (("one", (None, 0)), ("ws", (P(ws), nbytes)),
                             ("short", (P(ws), nbytes - 1))):
        y = torch.empty(M, N, dtype=xd.dtype, device="cuda")
        yr = torch.empty_like(y)
        h, yn = torch.empty_like(y), torch.empty_like(y)
        if mode == "one":
            _kparts_call("mi_qmm_affine", P(xd), P(w), P(s), P(b), P(y), M, N, K, 64, bits, dt)
            _kparts_call("mi_qmm_affine_residual", P(xd), P(w), P(s), P(b), P(rd), P(yr), M, N, K,
                         64, bits, dt)
            _kparts_call("mi_qmm_affine_residual_rmsnorm", P(xd), P(w), P(s), P(b), P(rd), P(nwd),
                         1e-6, P(h), P(yn), M, N, K, 64, bits, dt)
        else:
            _kparts_call("mi_qmm_affine_ws", P(xd), P(w), P(s), P(b), P(y), M, N, K, 64, bits, dt,
                         wsp, wsb)
            _kparts_call("mi_qmm_affine_residual_ws", P(xd), P(w), P(s), P(b), P(rd), P(yr), M, N,
                         K, 64, bits, dt, wsp, wsb)
            _kparts_call("mi_qmm_affine_residual_rmsnorm_ws", P(xd), P(w), P(s), P(b), P(rd),
                         P(nwd), 1e-6, P(h), P(yn), M, N, K, 64, bits, dt, wsp, wsb)
        torch.cuda.synchronize()
        ys[mode] = (y, yr, h, yn)
    for mode in ("ws", "short"):
        for a, c, what in zip(ys["one"], ys[mode], ("qmm", "qmm+add", "h", "rms_norm(h)")):
            assert torch.equal(a, c), f"{mode}: {what} differs from the one-launch entry"
    y, yr, h, yn = ys["ws"]
    want = oracle.quantized_matmul(x, *q, 64, bits, dtype)
    _close(y, want, dtype)
    _close(yr, oracle.round_to(res.astype(np.float64) + want, dtype), dtype)
    assert torch.equal(yr, h)
    _close(yn, oracle.rms_norm(to_np(h), nw, 1e-6, dtype), dtype)
    # the ops layer takes the workspace path: same bits
    assert torch.equal(ops.quantized_matmul(xd, w, s, b, group_size=64, bits=bits), y)


def test_qmm_k_parts_workspace_size():
    """The split rule is a function of (M, K): 8 < M <= 128 and K >= 4096 on
    the 16-bit MFMA path; N must be a multiple of 4."""
    L = hip.lib()
    bf = hip._DT[torch.bfloat16]
    assert L.mi_qmm_workspace_bytes(128, 2560, 4096, 64, 4, bf) == 4 * 128 * 2560 * 4
    assert L.mi_qmm_workspace_bytes(128, 2560, 9728, 64, 4, bf) == 4 * 128 * 2560 * 4
    assert L.mi_qmm_workspace_bytes(9, 64, 8192, 64, 8, bf) == 4 * 9 * 64 * 4
    for M, N, K, dt in ((8, 2560, 4096, bf), (129, 2560, 4096, bf), (128, 9728, 2560, bf),
                        (128, 2562, 4096, bf), (128, 2560, 4096, hip._DT[torch.float32])):
        assert L.mi_qmm_workspace_bytes(M, N, K, 64, 4, dt) == 0


@pytest.mark.parametrize("M", [100, 128])
def test_k_parts_multi_part_epilogues_equal_their_op_streams(M):
    """Dual, SwiGLU, split(3) and grouped q/k/v at K = 4096 run the parts in
    turn inside one launch; each equals, bit for bit, the op stream built from
    single-part quantized matmuls (which take the workspace path)."""
    r = rng(950 + M)
    K = 4096
    x = oracle.round_to(r.normal(0, 1, (1, M, K)), "bfloat16")
    xd = to_torch(x, "bfloat16")
    q1, q3 = _quant(951, 256, K), _quant(952, 256, K)
    w1, w3 = _dev(*q1, "bfloat16"), _dev(*q3, "bfloat16")
    g, u = ops.qmm_dual(xd, *w1, *w3)
    assert torch.equal(g, ops.quantized_matmul(xd, *w1))
    assert torch.equal(u, ops.quantized_matmul(xd, *w3))
    assert torch.equal(ops.qmm_dual(xd, *w1, *w3, swiglu=True), ops.swiglu(g, u))
    _close(g, oracle.quantized_matmul(x, *q1, 64, 4, "bfloat16"), "bfloat16")
    q = _quant(953, 3 * 128, K)
    wq = _dev(*q, "bfloat16")
    c, bx = ops.qmm_split_gate(xd, *wq)
    full = ops.quantized_matmul(xd, *wq)
    assert torch.equal(c, full[..., 128:256])
    assert torch.equal(bx, (full[..., :128].float() * full[..., 256:].float()).to(torch.bfloat16))
    qs = [_quant(954 + i, n, K) for i, n in enumerate((256, 64, 96))]
    wg = [_dev(*qq, "bfloat16") for qq in qs]
    for y, ww in zip(ops.qmm_grouped3(xd, wg), wg):
        assert torch.equal(y, ops.quantized_matmul(xd, *ww))


@pytest.mark.parametrize("M", [1, 100, 300])
def test_qmm_split_gate(M):
    r = rng(600 + M)
    K, D = 1024, 256
    x = oracle.round_to(r.normal(0, 1, (1, M, K)), "bfloat16")
    wq, s, b = _quant(17, 3 * D, K)
    c, bx = ops.qmm_split_gate(to_torch(x, "bfloat16"), *_dev(wq, s, b, "bfloat16"))
    full = oracle.quantized_matmul(x, wq, s, b, 64, 4, "bfloat16")
    c_want, bx_want = oracle.split_gate(full, "bfloat16")
    _close(c, c_want, "bfloat16")
    _close(bx, bx_want, "bfloat16")


@pytest.mark.parametrize("M", [1, 20, 128, 300, 600])
def test_qmm_dual_and_swiglu(M):
    r = rng(700 + M)
    K, N = 1024, 384
    x = oracle.round_to(r.normal(0, 1, (1, M, K)), "bfloat16")
    q1 = _quant(18, N, K)
    q3 = _quant(19, N, K)
    xd = to_torch(x, "bfloat16")
    g, u = ops.qmm_dual(xd, *_dev(*q1, "bfloat16"), *_dev(*q3, "bfloat16"))
    gw = oracle.quantized_matmul(x, *q1, 64, 4, "bfloat16")
    uw = oracle.quantized_matmul(x, *q3, 64, 4, "bfloat16")
    _close(g, gw, "bfloat16")
    _close(u, uw, "bfloat16")
    sw = ops.qmm_dual(xd, *_dev(*q1, "bfloat16"), *_dev(*q3, "bfloat16"), swiglu=True)
    _close(sw, oracle.swiglu(gw, uw, "bfloat16"), "bfloat16")
    # fused epilogue == swiglu of the unfused outputs, bit for bit
    assert torch.equal(sw, ops.swiglu(g, u))
    # either output equals the single-weight launch, bit for bit
    assert torch.equal(g, ops.quantized_matmul(xd, *_dev(*q1, "bfloat16")))
    assert torch.equal(u, ops.quantized_matmul(xd, *_dev(*q3, "bfloat16")))


@pytest.mark.parametrize("K", [128, 256, 640, 2048])
@pytest.mark.parametrize("bits", [4, 8])
def test_qmm_interleaved_k_split(K, bits):
    """From M = 512 the four K-split waves take interleaved stages (wave w:
    stages w, w + 4, ...) with one scale/bias table for the workgroup; at
    K = 128 two waves have no stage of their own, at K = 640 the waves take
    3, 3, 2 and 2 stages. Within tolerance of the
    oracle, with the residual epilogue, and row-independent: the last rows
    of an M = 520 launch equal, bit for bit, the same rows leading an
    M = 600 launch (other tiles, the same order)."""
    M, N = 520, 256
    r = rng(1400 + K + bits)
    x = oracle.round_to(r.normal(0, 1, (1, M, K)), "bfloat16")
    res = oracle.round_to(r.normal(0, 1, (1, M, N)), "bfloat16")
    q = _quant(1401 + K, N, K, bits=bits)
    xd, rd, w = to_torch(x, "bfloat16"), to_torch(res, "bfloat16"), _dev(*q, "bfloat16")
    y = ops.quantized_matmul(xd, *w, bits=bits)
    t = oracle.quantized_matmul(x, *q, 64, bits, "bfloat16")
    _close(y, t, "bfloat16")
    yr = ops.qmm_residual(xd, *w, rd, bits=bits)
    _close(yr, oracle.round_to(res.astype(np.float64) + t, "bfloat16"), "bfloat16")
    ext = torch.cat([xd[:, 500:], xd[:, :580]], dim=1).contiguous()  # M = 600
    assert torch.equal(y[:, 500:], ops.quantized_matmul(ext, *w, bits=bits)[:, :20])


@pytest.mark.parametrize("M,N", [(128, 9728), (100, 9728), (128, 8704), (128, 5120)])
def test_qmm_dual_mixed_tiles_equal_plain_tiles(M, N):
    """64 < M <= 128 whose 64-token grid puts one workgroup more on some CUs
    runs a mixed grid. On MI355X's 256 CUs, N = 9728 (304 feature tiles) and
    N = 8704 (272) take 128-token tiles for the first feature tiles, 64-token
    pairs after them and 32-token quarters for the last ones; N = 5120 (160)
    takes 64-token pairs and 32-token quads. Tiles never change results, so
    it equals, bit for bit, rows [0, 64) and [64, M) from two launches of at
    most 64 rows (the plain 64-token grid); every output element is written
    (a NaN-filled output comes back equal); and features at both ends (the
    first and last tile kinds) are within tolerance of the oracle."""
    r = rng(760 + M + N)
    K = 2560
    x = oracle.round_to(r.normal(0, 1, (1, M, K)), "bfloat16")
    q1 = _quant(761, N, K)
    q3 = _quant(762, N, K)
    xd = to_torch(x, "bfloat16")
    w = (*_dev(*q1, "bfloat16"), *_dev(*q3, "bfloat16"))
    lo_x, hi_x = xd[:, :64].contiguous(), xd[:, 64:].contiguous()
    g, u = ops.qmm_dual(xd, *w)
    for full, part_lo, part_hi in zip((g, u), ops.qmm_dual(lo_x, *w), ops.qmm_dual(hi_x, *w)):
        assert torch.equal(full, torch.cat([part_lo, part_hi], dim=1))
    sw = ops.qmm_dual(xd, *w, swiglu=True)
    sw_parts = [ops.qmm_dual(part, *w, swiglu=True) for part in (lo_x, hi_x)]
    assert torch.equal(sw, torch.cat(sw_parts, dim=1))
    # every tile of the grid is written: a NaN-filled output comes back whole
    poisoned = torch.full_like(sw, float("nan"))
    hip.b_qmm_dual([xd, *w], [poisoned], {**ops._qp(64, 4), "act": hip.MI_ACT_SWIGLU})
    assert torch.equal(poisoned, sw)
    for sl in (slice(0, 256), slice(N - 256, N)):
        gw = oracle.quantized_matmul(x, *(a[sl] for a in q1), 64, 4, "bfloat16")
        uw = oracle.quantized_matmul(x, *(a[sl] for a in q3), 64, 4, "bfloat16")
        _close(g[..., sl], gw, "bfloat16")
        _close(u[..., sl], uw, "bfloat16")
        _close(sw[..., sl], oracle.swiglu(gw, uw, "bfloat16"), "bfloat16")


@pytest.mark.parametrize("M,N", [(128, 9728), (100, 9728), (128, 10240)])
def test_qmm_wide_single_part_tiles(M, N):
    """A wide single-part 4-bit output at M = 128 runs 64-feature x 128-token
    tiles (N = 9728: 152 workgroups), M = 100 the 32 x 64 grid. Tiles never
    change results: either equals, bit for bit, rows [0, 64) and [64, M)
    from launches of at most 64 rows, with and without the residual
    epilogue; every element is written (NaN-filled output); and both ends
    are within tolerance of the oracle."""
    r = rng(880 + M + N)
    K = 2560
    x = oracle.round_to(r.normal(0, 1, (1, M, K)), "bfloat16")
    q = _quant(881, N, K)
    xd = to_torch(x, "bfloat16")
    w = _dev(*q, "bfloat16")
    res = to_torch(oracle.round_to(r.normal(0, 1, (1, M, N)), "bfloat16"), "bfloat16")
    y = ops.quantized_matmul(xd, *w)
    parts = [ops.quantized_matmul(xd[:, sl].contiguous(), *w) for sl in (slice(0, 64), slice(64, M))]
    assert torch.equal(y, torch.cat(parts, dim=1))
    yr = ops.qmm_residual(xd, *w, res)
    rparts = [ops.qmm_residual(xd[:, sl].contiguous(), *w, res[:, sl].contiguous())
              for sl in (slice(0, 64), slice(64, M))]
    assert torch.equal(yr, torch.cat(rparts, dim=1))
    poisoned = torch.full_like(y, float("nan"))
    hip.b_qmm([xd, *w], [poisoned], ops._qp(64, 4))
    assert torch.equal(poisoned, y)
    for sl in (slice(0, 256), slice(N - 256, N)):
        want = oracle.quantized_matmul(x, *(a[sl] for a in q), 64, 4, "bfloat16")
        _close(y[..., sl], want, "bfloat16")


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_qmm_dual_8bit_large_tiles(dtype):
    """The 8-bit dual from M = 512 runs 128-token tiles whose x offsets are
    rebuilt per stage (M = 520: a last tile of 8 tokens, whose other 120 rows
    read zeros past the end of x). Within tolerance of the oracle; rows
    [0, 512) equal, bit for bit, a launch of M = 512, and the ragged rows
    [480, 520) the first 40 rows of a launch of M = 552 that starts with
    them (whole tiles there; every M from 512 adds K in the same interleaved
    order, smaller M in contiguous chunks); every element written (NaN-filled
    output); the fused SwiGLU equals swiglu of the unfused pair bit for bit."""
    M, N, K = 520, 512, 1024
    r = rng(790)
    x = oracle.round_to(r.normal(0, 1, (1, M, K)), dtype)
    q1 = _quant(791, N, K, bits=8, dtype=dtype)
    q3 = _quant(792, N, K, bits=8, dtype=dtype)
    xd = to_torch(x, dtype)
    w = (*_dev(*q1, dtype), *_dev(*q3, dtype))
    g, u = ops.qmm_dual(xd, *w, bits=8)
    gw = oracle.quantized_matmul(x, *q1, 64, 8, dtype)
    uw = oracle.quantized_matmul(x, *q3, 64, 8, dtype)
    _close(g, gw, dtype)
    _close(u, uw, dtype)
    pg, pu = ops.qmm_dual(xd[:, :512].contiguous(), *w, bits=8)
    assert torch.equal(g[:, :512], pg) and torch.equal(u[:, :512], pu)
    ext = torch.cat([xd[:, 480:520], xd[:, :512]], dim=1).contiguous()  # M = 552
    pg, pu = ops.qmm_dual(ext, *w, bits=8)
    assert torch.equal(g[:, 480:520], pg[:, :40]) and torch.equal(u[:, 480:520], pu[:, :40])
    sw = ops.qmm_dual(xd, *w, bits=8, swiglu=True)
    assert torch.equal(sw, ops.swiglu(g, u))
    _close(sw, oracle.swiglu(gw, uw, dtype), dtype)
    poisoned = torch.full_like(sw, float("nan"))
    hip.b_qmm_dual([xd, *w], [poisoned], {**ops._qp(64, 8), "act": hip.MI_ACT_SWIGLU})
    assert torch.equal(poisoned, sw)


@pytest.mark.parametrize("M", [1, 3, 8, 16, 40, 128, 300, 520])
@pytest.mark.parametrize("bits,dtype", [(4, "bfloat16"), (8, "float16"), (4, "float32")])
def test_qmm_grouped3_equals_three_launches(M, bits, dtype):
    """q/k/v in one launch: bit-identical to three mi_qmm_affine calls (the
    per-element reduction order does not depend on the tile), and within the
    tolerance of the oracle; parts of unequal width (4096-like / 1024-like)."""
    r = rng(720 + M + bits)
    K = 512
    Ns = (256, 64, 96)
    x = oracle.round_to(r.normal(0, 1, (1, M, K)), dtype)
    qs = [_quant(721 + i, n, K, 64, bits, dtype) for i, n in enumerate(Ns)]
    xd = to_torch(x, dtype)
    ws = [_dev(*q, dtype) for q in qs]
    got = ops.qmm_grouped3(xd, ws, 64, bits)
    for (wq, s, b), w, y in zip(qs, ws, got):
        sep = ops.quantized_matmul(xd, *w, group_size=64, bits=bits)
        assert torch.equal(y, sep)
        _close(y, oracle.quantized_matmul(x, wq, s, b, 64, bits, dtype), dtype,
               1e-5 if dtype == "float32" else None)


@pytest.mark.parametrize("M", [128, 72])
def test_qmm_grouped3_mixed_tiles_qwen3_shape(M):
    """Qwen3 q/k/v (N 4096 + 1024 + 1024, K 2560) at 64 < M <= 128, where the
    grouped launch and the three separate launches use different grids: bit
    for bit equal, and within tolerance of the oracle on the first and last
    128 features of each part."""
    r = rng(740 + M)
    K = 2560
    Ns = (4096, 1024, 1024)
    x = oracle.round_to(r.normal(0, 1, (1, M, K)), "bfloat16")
    qs = [_quant(741 + i, n, K) for i, n in enumerate(Ns)]
    xd = to_torch(x, "bfloat16")
    ws = [_dev(*q, "bfloat16") for q in qs]
    got = ops.qmm_grouped3(xd, ws, 64, 4)
    for q, w, y in zip(qs, ws, got):
        assert torch.equal(y, ops.quantized_matmul(xd, *w, group_size=64, bits=4))
        n = q[0].shape[0]
        for sl in (slice(0, 128), slice(n - 128, n)):
            want = oracle.quantized_matmul(x, *(a[sl] for a in q), 64, 4, "bfloat16")
            _close(y[..., sl], want, "bfloat16")


@pytest.mark.parametrize("Ns,bits", [((256, 64, 128), 4), ((256, 96, 64), 4), ((128, 64, 64), 8)])
def test_qmm_grouped3_large_m_tiles(Ns, bits):
    """From M = 512 the grouped launch takes 64-feature tiles when every part
    is a multiple of 64, else 32-feature tiles: both bit for bit equal to the
    three separate launches (which take their own tiles), and within the
    oracle's tolerance on the first rows."""
    r = rng(760 + sum(Ns) + bits)
    M, K = 520, 512
    x = oracle.round_to(r.normal(0, 1, (1, M, K)), "bfloat16")
    qs = [_quant(761 + i, n, K, 64, bits) for i, n in enumerate(Ns)]
    xd = to_torch(x, "bfloat16")
    ws = [_dev(*q, "bfloat16") for q in qs]
    got = ops.qmm_grouped3(xd, ws, 64, bits)
    for q, w, y in zip(qs, ws, got):
        assert torch.equal(y, ops.quantized_matmul(xd, *w, group_size=64, bits=bits))
        want = oracle.quantized_matmul(x[:, :64], *q, 64, bits, "bfloat16")
        _close(y[:, :64], want, "bfloat16")


def test_qmm_grouped3_rejects_unaligned_parts():
    K = 256
    qs = [_quant(730 + i, n, K) for i, n in enumerate((64, 48, 64))]
    x = to_torch(np.zeros((1, 4, K), np.float32), "bfloat16")
    with pytest.raises(ValueError, match="multiple of 32"):
        ops.qmm_grouped3(x, [_dev(*q, "bfloat16") for q in qs])


# ------------------------------------------------------------------ A5-A10


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("D", [2560, 2048, 100])
def test_rms_norm(dtype, D):
    r = rng(800 + D)
    x = oracle.round_to(r.normal(0, 1, (3, 37, D)), dtype)
    w = oracle.round_to(1 + 0.2 * r.normal(0, 1, D), dtype)
    y = ops.rms_norm(to_torch(x, dtype), to_torch(w, dtype), 1e-6)
    _close(y, oracle.rms_norm(x, w, 1e-6, dtype), dtype, 1e-5 if dtype == "float32" else None)


def test_rms_norm_eps_placement_gpu():
    x = np.full((2, 32), 0.5, np.float32)
    y = to_np(ops.rms_norm(to_torch(x, "float32"), to_torch(np.full(32, 1.5, np.float32), "float32"), 0.25))
    assert y[0, 0] == pytest.approx(1.5 * 0.5 / math.sqrt(0.5), rel=1e-6)


@pytest.mark.parametrize("H,D,L,offset,norm", [(32, 128, 128, 0, True), (8, 128, 1, 128, True),
                                                (32, 64, 64, 5, True), (4, 128, 7, 0, False)])
def test_norm_rope(H, D, L, offset, norm):
    r = rng(900 + H + D + L)
    x = oracle.round_to(r.normal(0, 1, (1, L, H * D)), "bfloat16")
    w = oracle.round_to(1 + 0.2 * r.normal(0, 1, D), "bfloat16") if norm else None
    got = ops.norm_rope(to_torch(x, "bfloat16"), None if w is None else to_torch(w, "bfloat16"),
                        H, 1e-6, D, 1e6, offset)
    want = oracle.norm_rope(x, w, 1e-6, H, D, 1e6, offset, "bfloat16")
    _close(got, want, "bfloat16")


@pytest.mark.parametrize("D", [64, 128])
def test_norm_rope_norm_only(D):
    """rope dims 0 with a norm weight: the q/k RMSNorm alone (16-byte rows:
    eight consecutive elements per lane)."""
    r = rng(905 + D)
    H, L = 8, 9
    x = oracle.round_to(r.normal(0, 1, (1, L, H * D)), "bfloat16")
    w = oracle.round_to(1 + 0.2 * r.normal(0, 1, D), "bfloat16")
    got = ops.norm_rope(to_torch(x, "bfloat16"), to_torch(w, "bfloat16"), H, 1e-6, 0, 1e6, 0)
    _close(got, oracle.norm_rope(x, w, 1e-6, H, 0, 1e6, 0, "bfloat16"), "bfloat16")


@pytest.mark.parametrize("dims", [128, 0])
def test_norm_rope_unaligned_rows(dims):
    """Rows whose stride is not a multiple of 8 elements take the one-pair-per-
    lane form (and the general loop for dims 0); both stay within the oracle
    bar, and within it of the 16-byte-row form on the same values."""
    r = rng(915 + dims)
    H, D, L, offset = 8, 128, 11, 3
    x = oracle.round_to(r.normal(0, 1, (1, L, H * D)), "bfloat16")
    w = oracle.round_to(1 + 0.2 * r.normal(0, 1, D), "bfloat16")
    pad = torch.zeros((1, L, H * D + 4), dtype=torch.bfloat16, device="cuda")
    pad[:, :, :H * D] = to_torch(x, "bfloat16")
    wd = to_torch(w, "bfloat16")
    out = torch.empty((1, H, L, D), dtype=torch.bfloat16, device="cuda")
    hip._check(hip.lib().mi_norm_rope(
        pad.data_ptr(), wd.data_ptr(), out.data_ptr(), 1, L, H, D, H * D + 4, 1e-6, dims, 0, 1e6,
        1.0, offset, L, 0, hip._dt(pad), torch.cuda.current_stream().cuda_stream), "norm_rope")
    want = oracle.norm_rope(x, w, 1e-6, H, dims, 1e6, offset, "bfloat16")
    _close(out, want, "bfloat16")
    vec = ops.norm_rope(to_torch(x, "bfloat16"), wd, H, 1e-6, dims, 1e6, offset)
    _close(out, to_np(vec), "bfloat16")


def test_rope_partial_traditional_fp32():
    r = rng(950)
    x = r.normal(0, 1, (2, 3, 9, 32)).astype(np.float32)
    for trad in (False, True):
        got = ops.rope(to_torch(x, "float32"), 24, traditional=trad, base=1e4, offset=11)
        _close(got, oracle.rope(x, 24, trad, 1e4, 1.0, 11, "float32"), "float32", 2e-5)


def test_norm_rope_into_cache():
    r = rng(960)
    H, D, cap = 8, 128, 64
    x = oracle.round_to(r.normal(0, 1, (1, 5, H * D)), "bfloat16")
    cache = torch.full((1, H, cap, D), 7.0, dtype=torch.bfloat16, device="cuda")
    ops.norm_rope(to_torch(x, "bfloat16"), None, H, 0.0, D, 1e6, 10, out=cache, out_pos=10)
    want = oracle.norm_rope(x, None, 0.0, H, D, 1e6, 10, "bfloat16")
    c = to_np(cache)
    _close(c[:, :, 10:15], want, "bfloat16")
    assert (c[:, :, :10] == 7.0).all() and (c[:, :, 15:] == 7.0).all()


@pytest.mark.parametrize("L,offset,strided", [(128, 0, False), (1, 128, False), (7, 3, True)])
def test_norm_rope_qkv_equals_three_calls(L, offset, strided):
    """The one-launch attention prologue == q norm_rope + k norm_rope into the
    cache + v cache write, bit for bit; q/k/v may be column slices of one
    [B, L, (H + 2 HK) D] buffer (row stride > H D); cache rows outside
    [offset, offset + L) stay untouched."""
    r = rng(970 + L)
    H, HK, D, cap = 32, 8, 128, 160
    qkv = oracle.round_to(r.normal(0, 1, (1, L, (H + 2 * HK) * D)), "bfloat16")
    qn = oracle.round_to(1 + 0.2 * r.normal(0, 1, D), "bfloat16")
    kn = oracle.round_to(1 + 0.2 * r.normal(0, 1, D), "bfloat16")
    t = to_torch(qkv, "bfloat16")
    if strided:
        q, k, v = t[..., :H * D], t[..., H * D:(H + HK) * D], t[..., (H + HK) * D:]
    else:
        q, k, v = (t[..., :H * D].contiguous(), t[..., H * D:(H + HK) * D].contiguous(),
                   t[..., (H + HK) * D:].contiguous())
    qw, kw = to_torch(qn, "bfloat16"), to_torch(kn, "bfloat16")
    kc = torch.full((1, HK, cap, D), 5.0, dtype=torch.bfloat16, device="cuda")
    vc = torch.full_like(kc, 6.0)
    qr = ops.norm_rope_qkv(q, k, v, qw, kw, H, HK, 1e-6, D, 1e6, offset, kc, vc, offset)
    kc2, vc2 = torch.full_like(kc, 5.0), torch.full_like(kc, 6.0)
    qr2 = ops.norm_rope(q.contiguous(), qw, H, 1e-6, D, 1e6, offset)
    ops.norm_rope(k.contiguous(), kw, HK, 1e-6, D, 1e6, offset, out=kc2, out_pos=offset)
    ops.write_kv(v.contiguous(), HK, vc2, offset)
    assert torch.equal(qr, qr2) and torch.equal(kc, kc2) and torch.equal(vc, vc2)
    _close(qr, oracle.norm_rope(qkv[..., :H * D], qn, 1e-6, H, D, 1e6, offset, "bfloat16"),
           "bfloat16")
    assert (to_np(kc)[:, :, offset + L:] == 5.0).all() and (to_np(vc)[:, :, :offset] == 6.0).all()


@pytest.mark.parametrize("H,HK,Lq,Lk,D,causal", [(32, 8, 128, 128, 128, True),
                                                 (32, 8, 1, 129, 128, True),
                                                 (32, 8, 200, 200, 64, True),
                                                 (8, 8, 40, 70, 64, True),
                                                 (6, 2, 33, 33, 128, False),
                                                 (12, 4, 5, 130, 128, True),
                                                 (32, 8, 512, 512, 64, True),      # shared-K/V kernel
                                                 (16, 2, 1000, 1030, 128, True)])  # shared, 2 quads
def test_sdpa(H, HK, Lq, Lk, D, causal):
    r = rng(1000 + Lq + Lk + D)
    q = oracle.round_to(r.normal(0, 1, (1, H, Lq, D)), "bfloat16")
    k = oracle.round_to(r.normal(0, 1, (1, HK, Lk, D)), "bfloat16")
    v = oracle.round_to(r.normal(0, 1, (1, HK, Lk, D)), "bfloat16")
    scale = D ** -0.5
    want = oracle.sdpa(q, k, v, scale, causal, "bfloat16")
    o = ops.scaled_dot_product_attention(to_torch(q, "bfloat16"), to_torch(k, "bfloat16"),
                                         to_torch(v, "bfloat16"), scale, "causal" if causal else None)
    _close(o, want, "bfloat16")
    o1 = ops.scaled_dot_product_attention(to_torch(q, "bfloat16"), to_torch(k, "bfloat16"),
                                          to_torch(v, "bfloat16"), scale,
                                          "causal" if causal else None, out_layout=1)
    assert torch.equal(o1, o.transpose(1, 2).contiguous())


@pytest.mark.parametrize("H,HK,L,D,causal", [(32, 8, 512, 64, True), (16, 2, 1024, 128, True),
                                             (32, 8, 512, 128, False), (32, 8, 544, 64, False)])
def test_sdpa_shared_and_split_kernels_agree(H, HK, L, D, causal):
    """A row's attention is the same bits whichever kernel computes it. The
    L-row call runs the shared-K/V kernel (a grid of at least 128
    workgroups, causal q blocks paired long with short); a call on its last
    32 query rows, and a decode call on its last row, run the key-split
    kernel (smaller grids) over the same keys. Causal at head dim 64, the q
    blocks with 1, 2, 3, 5 and 8 key tiles (fewer streams than four, streams
    of unequal length) are also checked against split-kernel calls over
    their own visible keys. L = 544 (17 tiles, no mask, an odd block count:
    no pairing) gives stream 0 one tile more than the others."""
    r = rng(1050 + L + D)
    q = to_torch(oracle.round_to(r.normal(0, 1, (1, H, L, D)), "bfloat16"), "bfloat16")
    k = to_torch(oracle.round_to(r.normal(0, 1, (1, HK, L, D)), "bfloat16"), "bfloat16")
    v = to_torch(oracle.round_to(r.normal(0, 1, (1, HK, L, D)), "bfloat16"), "bfloat16")
    mask = "causal" if causal else None
    full = ops.scaled_dot_product_attention(q, k, v, D ** -0.5, mask)
    tail = ops.scaled_dot_product_attention(q[:, :, L - 32:].contiguous(), k, v, D ** -0.5, mask)
    last = ops.scaled_dot_product_attention(q[:, :, L - 1:].contiguous(), k, v, D ** -0.5, mask)
    assert torch.equal(full[:, :, L - 32:], tail)
    assert torch.equal(full[:, :, L - 1:], last)
    if causal and D == 64:
        for j in (0, 1, 2, 4, 7):
            rows = slice(32 * j, 32 * j + 32)
            part = ops.scaled_dot_product_attention(q[:, :, rows].contiguous(),
                                                    k[:, :, :32 * j + 32].contiguous(),
                                                    v[:, :, :32 * j + 32].contiguous(),
                                                    D ** -0.5, mask)
            assert torch.equal(full[:, :, rows], part), f"q block {j}"


def test_sdpa_kv_cache_capacity():
    """Only the first kv_len rows of a larger cache are read."""
    r = rng(1100)
    q = oracle.round_to(r.normal(0, 1, (1, 4, 3, 64)), "bfloat16")
    k = oracle.round_to(r.normal(0, 1, (1, 2, 40, 64)), "bfloat16")
    v = oracle.round_to(r.normal(0, 1, (1, 2, 40, 64)), "bfloat16")
    kd, vd = to_torch(k, "bfloat16"), to_torch(v, "bfloat16")
    kd[:, :, 20:] = float("nan")
    vd[:, :, 20:] = float("nan")
    o = ops.scaled_dot_product_attention(to_torch(q, "bfloat16"), kd, vd, 0.125, "causal", kv_len=20)
    _close(o, oracle.sdpa(q, k[:, :, :20], v[:, :, :20], 0.125, True, "bfloat16"), "bfloat16")


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("n", [128 * 9728, 1001])
def test_swiglu(dtype, n):
    r = rng(1200)
    g = oracle.round_to(r.normal(0, 2, n), dtype)
    u = oracle.round_to(r.normal(0, 1, n), dtype)
    y = ops.swiglu(to_torch(g, dtype), to_torch(u, dtype))
    _close(y, oracle.swiglu(g, u, dtype), dtype, 1e-5 if dtype == "float32" else None)


@pytest.mark.parametrize("L,with_state", [(2048, False), (1, True), (5, True)])
def test_shortconv(L, with_state):
    r = rng(1300 + L)
    B, D = 1, 2048
    bx = oracle.round_to(r.normal(0, 1, (B, L, D)), "bfloat16")
    c = oracle.round_to(r.normal(0, 1, (B, L, D)), "bfloat16")
    w = oracle.round_to(r.normal(0, 0.5, (D, 3)), "bfloat16")
    st = oracle.round_to(r.normal(0, 1, (B, 2, D)), "bfloat16") if with_state else None
    out, st_out = ops.shortconv(to_torch(bx, "bfloat16"), to_torch(c, "bfloat16"),
                                to_torch(w, "bfloat16"), None if st is None else to_torch(st, "bfloat16"))
    want, st_want = oracle.shortconv(bx, c, w, st, "bfloat16")
    _close(out, want, "bfloat16")
    assert np.array_equal(to_np(st_out), st_want)
    # the scalar path (bx one element off 16-byte alignment) gives the same bits
    flat = to_torch(np.concatenate([[0.0], bx.reshape(-1)]).astype(np.float32), "bfloat16")
    bx_odd = flat[1:].reshape(B, L, D)
    out2, st_out2 = ops.shortconv(bx_odd, to_torch(c, "bfloat16"), to_torch(w, "bfloat16"),
                                  None if st is None else to_torch(st, "bfloat16"))
    assert torch.equal(out, out2) and torch.equal(st_out, st_out2)


def test_linear_gelu_f32():
    r = rng(1400)
    x = r.normal(0, 1, (32, 256)).astype(np.float32)
    w1 = r.normal(0, 0.02, (1024, 256)).astype(np.float32)
    b1 = r.normal(0, 0.1, 1024).astype(np.float32)
    h = ops.linear_f32(to_torch(x, "float32"), to_torch(w1, "float32"), to_torch(b1, "float32"), gelu=True)
    want = oracle.gelu(x.astype(np.float64) @ w1.T.astype(np.float64) + b1).astype(np.float32)
    _close(h, want, "float32", 1e-5)


def _mlp_inputs(seed, M, K, H, N, biases=True):
    r = rng(seed)
    x = r.normal(0, 1, (M, K)).astype(np.float32)
    w1 = r.normal(0, 0.02, (H, K)).astype(np.float32)
    w2 = r.normal(0, 0.02, (N, H)).astype(np.float32)
    b1 = (r.normal(0, 0.1, H) if biases else np.zeros(H)).astype(np.float32)
    b2 = (r.normal(0, 0.1, N) if biases else np.zeros(N)).astype(np.float32)
    return x, w1, b1, w2, b2


@pytest.mark.parametrize("M,K,H,N,biases", [
    (32, 256, 1024, 256, False),   # config 1: b = 0
    (32, 256, 1024, 256, True),
    (128, 256, 512, 256, True),    # the reference toy (examples/tiny_mlp.py:5-6)
    (37, 64, 1000, 72, True),      # ragged rows, a partial last hidden chunk
])
def test_tiny_mlp_region_one_launch(M, K, H, N, biases):
    """Config 1 as one region and one launch (regions.tiny_mlp through
    kernels.call), NaN-poisoned output, vs oracle.tiny_mlp at fp32 1e-5; three
    calls are bitwise identical (fixed-order reduction of the hidden chunks,
    the ticket counters reset by every call)."""
    from autotuner_runtime import kernels, regions

    host = _mlp_inputs(1410 + M, M, K, H, N, biases)
    ins = [to_torch(a, "float32") for a in host]
    spec = regions.tiny_mlp()
    runs = [kernels.call(spec, ins, init_value=float("nan"))[0] for _ in range(3)]
    torch.cuda.synchronize()
    assert not torch.isnan(runs[0]).any()
    assert all(torch.equal(runs[0], r) for r in runs[1:])
    want = oracle.tiny_mlp(*[a.astype(np.float64) for a in host])
    err = _close(runs[0], want, "float32", 1e-5)
    # the two-launch stream agrees within the same bar
    h = ops.linear_f32(ins[0], ins[1], ins[2], gelu=True)
    _close(ops.linear_f32(h, ins[3], ins[4]), want, "float32", 1e-5)
    print(f"\ntiny mlp {M}x{K}->{H}->{N}: max-abs-normalised error {err:.3e}")


def test_tiny_mlp_calls_of_different_sizes_share_the_workspace():
    """Back-to-back calls of different row counts on one stream (one cached
    workspace): each equals the oracle, so no ticket or partial leaks from one
    call into the next. The sizes 1000, 300, 600 in turn are the case where a
    ticket region sized by M let a smaller call's partial sums overwrite the
    counters a larger call reads (the prefix is now fixed)."""
    for i, (M, H) in enumerate(((32, 1024), (9, 256), (32, 1024), (1, 64),
                                (1000, 256), (300, 256), (600, 256))):
        host = _mlp_inputs(1450 + i, M, 256, H, 256)
        got = ops.gelu_mlp_f32(*[to_torch(a, "float32") for a in host])
        _close(got, oracle.tiny_mlp(*[a.astype(np.float64) for a in host]), "float32", 1e-5)


@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
def test_argmax_lowest_index_on_ties(dtype, split):
    """Ties across workgroup spans (4096 bf16 / 2048 f32 values per span on the
    split path) and across threads: the lowest index wins; NaN never wins."""
    r = rng(1500)
    x = oracle.round_to(r.normal(0, 1, (6, 151936)), dtype)
    x[1, 77] = x[1, 90000] = 50.0          # tie across spans
    x[2, :] = -1.0
    x[2, 5] = float("nan")                  # NaN never wins
    x[3, 4095] = x[3, 4096] = x[3, 2047] = 60.0  # ties at span edges: 2047 wins
    x[4, -1] = 70.0                         # maximum in the last element
    x[5, :2048] = np.nan                    # a whole NaN span, maximum after it
    x[5, 3000] = 80.0
    got = ops.argmax(to_torch(x, dtype), split=split).cpu().numpy()
    assert got.tolist() == [int(np.argmax(x[0])), 77, 0, 2047, 151935, 3000]


@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("V", [1, 7, 1001, 8 * 1024 * 8 + 8, 65536])
@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
def test_argmax_shapes_ties_nan_and_unaligned_rows(V, dtype, split):
    """Vector (16-byte chunks) and scalar paths: random rows, a tie placed in
    one thread's later chunk and another thread's earlier one, an all-NaN row
    (-> 0), an all -inf row (-> 0), and a misaligned view (scalar path)."""
    r = rng(1510 + V)
    x = oracle.round_to(r.normal(0, 1, (5, V)), dtype)
    if V > 16:
        x[1, V - 3] = x[1, 9] = 40.0
    x[2, :] = np.nan
    x[3, :] = -np.inf
    want = [int(np.argmax(x[0])), 9 if V > 16 else int(np.argmax(x[1])), 0, 0,
            int(np.argmax(x[4]))]
    got = ops.argmax(to_torch(x, dtype), split=split).cpu().numpy()
    assert got.tolist() == want
    flat = to_torch(np.concatenate([[0.0], x[4]]).astype(np.float32), dtype)
    assert int(ops.argmax(flat[1:].reshape(1, V), split=split).item()) == want[4]  # data_ptr + 1


def test_argmax_workspace_size_and_checks():
    """Workspace bytes: 8 per 2048-value span per row (a bound for every
    path); a short or misaligned workspace is rejected before any launch."""
    from autotuner_runtime import hip

    L = hip.lib()
    assert L.mi_argmax_workspace_bytes(1, 151936) == 8 * 75
    assert L.mi_argmax_workspace_bytes(3, 2048) == 24 and L.mi_argmax_workspace_bytes(0, 5) == 0
    x = torch.zeros((2, 4096), dtype=torch.bfloat16, device="cuda")
    o = torch.empty(2, dtype=torch.int32, device="cuda")
    ws = torch.empty(64, dtype=torch.uint8, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    assert L.mi_argmax(x.data_ptr(), o.data_ptr(), 2, 4096, hip.MI_BF16, ws.data_ptr(), 8, st) \
        == hip.MI_ERR_ARG
    assert L.mi_argmax(x.data_ptr(), o.data_ptr(), 2, 4096, hip.MI_BF16, ws.data_ptr() + 4, 60,
                       st) == hip.MI_ERR_ARG


def test_determinism_three_runs():
    """The reference's gate: three runs bitwise identical (ladder/child.py:419-428)."""
    r = rng(1600)
    x = to_torch(oracle.round_to(r.normal(0, 1, (128, 2560)), "bfloat16"), "bfloat16")
    dev = _dev(*_quant(20, 9728, 2560), "bfloat16")
    outs = [ops.quantized_matmul(x, *dev) for _ in range(3)]
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])


def test_reference_sequence_replays_library_ops():
    """A starter spec's recorded MLX calls replay through the library ops:
    LFM2's conv in_proj [quantized_matmul, split(3), mul] equals the fused
    split_gate region bit for bit (the region keeps T(B * x) of the unfused
    projection), and [rms_norm, rope, sdpa] equals the same ops called
    directly."""
    from autotuner_runtime import kernels
    from autotuner_runtime.kernels import KernelSpec

    def ref(i):
        return {"$": "ref", "i": i}

    def node(op, ins, outs, *args, **kw):
        return {"op": op, "in_arrays": ins, "out_arrays": outs,
                "args": {"$": "tuple", "items": list(args)}, "kwargs": kw}

    M, D, K = 48, 256, 512
    r = rng(1300)
    x = to_torch(oracle.round_to(r.normal(0, 1, (1, M, K)), "bfloat16"), "bfloat16")
    w = _dev(*_quant(1301, 3 * D, K), "bfloat16")
    conv_in = {"nodes": [
        node("mx.quantized_matmul", [0, 1, 2, 3], [4], ref(0), ref(1), ref(2), ref(3),
             transpose=True, group_size=64, bits=4),
        node("mx.split", [4], [5, 6, 7], ref(0), 3, axis=-1),
        node("array.__mul__", [5, 7], [8], ref(0), ref(1))],
        "input_ids": [0, 1, 2, 3], "output_ids": [6, 8]}
    spec = KernelSpec(kernel_id="seed_conv_in", name="seed_conv_in",
                      input_names=("in0", "in1", "in2", "in3"), output_names=("out0", "out1"),
                      source="// original sequence starter",
                      output_shapes=(("1", str(M), str(D)),) * 2,
                      output_dtypes=("bfloat16", "bfloat16"), reference_sequence=conv_in)
    c, bx = kernels.call(spec, [x, *w])
    fc, fbx = ops.qmm_split_gate(x, *w)
    assert torch.equal(c, fc) and torch.equal(bx, fbx)

    H, L, Dh = 4, 64, 128
    q = to_torch(oracle.round_to(r.normal(0, 1, (1, H, L, Dh)), "bfloat16"), "bfloat16")
    kv = to_torch(oracle.round_to(r.normal(0, 1, (1, H, L, Dh)), "bfloat16"), "bfloat16")
    nw = to_torch(oracle.round_to(r.normal(1, 0.1, (Dh,)), "bfloat16"), "bfloat16")
    attn = {"nodes": [
        node("mx.fast.rms_norm", [0, 2], [3], ref(0), ref(1), 1e-6),
        node("mx.fast.rope", [3], [4], ref(0), Dh, traditional=False, base=1e6, scale=1.0,
             offset=0),
        node("mx.fast.scaled_dot_product_attention", [4, 1, 1], [5], ref(0), ref(1), ref(2),
             scale=Dh ** -0.5, mask="causal")],
        "input_ids": [0, 1, 2], "output_ids": [5]}
    from autotuner_runtime.original_sequence import prepare_sequence
    (o,) = prepare_sequence(attn)([q, kv, nw])
    qr = ops.rope(ops.rms_norm(q, nw, 1e-6), Dh, False, 1e6, 1.0, 0)
    assert torch.equal(o, ops.scaled_dot_product_attention(qr, kv, kv, Dh ** -0.5, "causal"))
