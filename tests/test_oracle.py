"""Pins of the CPU oracle (oracle/) -- CPU only.

The reference stores no arithmetic golden vectors for this path (its parity
tests compare live against MLX on an Apple GPU), so each oracle function is
pinned here by closed forms, known-answer cases, invariants, two independent
restatements agreeing, and brute force on tiny inputs -- each chosen so a
plausible mistake (reversed nibble order, mul+add instead of fma, eps outside
the sqrt, a wrong rope sign or frequency, a transposed GQA map, an off-by-one
causal mask) fails. Plus the committed golden fixtures (tests/golden/).
"""

from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
from conftest import rng


@pytest.fixture(autouse=True)
def _lib(oracle_lib):
    return oracle_lib


# ---------------------------------------------------------------------- A1


def test_nibble_order_is_lsb_first():
    """value j of a word sits at bits 4j..4j+3 (lower.py:1199-1211)."""
    q = np.arange(8, dtype=np.uint32)
    word = sum(int(v) << (4 * j) for j, v in enumerate(q))
    wq = np.array([[word, 0, 0, 0, 0, 0, 0, 0]], dtype=np.uint32)  # K = 64, one group
    s = np.array([[2.0]], np.float32)
    b = np.array([[-3.0]], np.float32)
    W = oracle.dequantize(wq, s, b, 64, 4, "bfloat16")
    assert W[0, :8].tolist() == [-3.0, -1.0, 1.0, 3.0, 5.0, 7.0, 9.0, 11.0]
    assert (W[0, 8:] == -3.0).all()
    assert oracle.pack(oracle.unpack(wq, 4), 4).tolist() == wq.tolist()


def test_byte_order_is_lsb_first_at_8_bits():
    word = 1 | (2 << 8) | (250 << 16) | (255 << 24)
    wq = np.zeros((1, 16), np.uint32)
    wq[0, 0] = word
    W = oracle.dequantize(wq, np.ones((1, 1), np.float32), np.zeros((1, 1), np.float32), 64, 8,
                          "float32")
    assert W[0, :4].tolist() == [1.0, 2.0, 250.0, 255.0]


def test_dequant_is_one_fused_rounding():
    """fp32 scales: fma(s, q, b) differs from mul-then-add here, and the
    closed form is 3 * 2^-23 exactly."""
    s = np.float32(1.0 + 2.0 ** -23)
    wq = np.zeros((1, 8), np.uint32)
    wq[0, 0] = 3
    W = oracle.dequantize(wq, np.array([[s]]), np.array([[-3.0]], np.float32), 64, 4, "float32")
    assert W[0, 0] == np.float32(3 * 2.0 ** -23)
    mul_add = np.float32(np.float32(s * np.float32(3)) + np.float32(-3))
    assert mul_add != W[0, 0]


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("bits,gs", [(4, 64), (4, 32), (4, 128), (8, 64)])
def test_dequant_two_restatements_agree_bitwise(dtype, bits, gs):
    r = rng(11 + bits + gs)
    N, K = 24, 512
    w = r.normal(0, 0.02, (N, K)).astype(np.float32)
    wq, s, b = oracle.quantize_affine(w, gs, bits, dtype)
    a = oracle.dequantize(wq, s, b, gs, bits, dtype)
    c = oracle.dequantize_numpy(wq, s, b, gs, bits, dtype)
    assert np.array_equal(a.view(np.uint32), c.view(np.uint32))


def test_dequant_closed_forms():
    r = rng(3)
    wq = r.integers(0, 2 ** 32, (4, 16), dtype=np.uint64).astype(np.uint32)
    s = np.zeros((4, 2), np.float32)
    b = oracle.round_to(r.normal(0, 1, (4, 2)), "bfloat16")
    W = oracle.dequantize(wq, s, b, 64, 4, "bfloat16")
    assert (W == np.repeat(b, 64, axis=1)).all()          # s = 0 -> b exactly
    q = oracle.unpack(wq, 4)
    assert q.max() <= 15 and q.min() >= 0


def test_quantizer_round_trip_within_half_step():
    r = rng(5)
    w = r.normal(0, 0.02, (16, 256)).astype(np.float32)
    wq, s, b = oracle.quantize_affine(w, 64, 4, "float32")
    W = oracle.dequantize(wq, s, b, 64, 4, "float32")
    step = np.repeat(s, 64, axis=1)
    assert (np.abs(W - w) <= step * 0.5 + 1e-7).all()


def test_bf16_rounding_is_nearest_even():
    vals = np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -9, -1.0 - 2 ** -8], np.float32)
    got = oracle.round_to(vals, "bfloat16")
    assert got.tolist() == [1.0, 1.0 + 2 ** -6, 1.0, -1.0]


# ------------------------------------------------------------------- A2-A4


def _qmm_case(seed, M, N, K, gs=64, bits=4, dtype="bfloat16"):
    r = rng(seed)
    x = oracle.round_to(r.normal(0, 1, (M, K)), dtype)
    wq, s, b = oracle.quantize_affine(r.normal(0, 0.02, (N, K)).astype(np.float32), gs, bits, dtype)
    return x, wq, s, b


def test_qmm_zero_input_is_exactly_zero():
    x, wq, s, b = _qmm_case(1, 3, 32, 256)
    x[:] = 0
    assert (oracle.qmm_factored(x, wq, s, b, 64, 4, "bfloat16") == 0).all()
    assert (oracle.quantized_matmul(x, wq, s, b, 64, 4, "bfloat16") == 0).all()


def test_qmm_zero_scales_give_bias_times_group_sums():
    x, wq, s, b = _qmm_case(2, 4, 16, 256, dtype="float32")
    s[:] = 0
    want = np.einsum("mgk,ng->mn", x.reshape(4, 4, 64).astype(np.float64), b.astype(np.float64))
    got = oracle.qmm_factored(x, wq, s, b, 64, 4, "float32")
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("bits", [4, 8])
def test_qmm_one_hot_rows_select_dequantized_columns(bits):
    x, wq, s, b = _qmm_case(3, 5, 48, 256, bits=bits)
    x[:] = 0
    cols = [0, 7, 63, 64, 255]
    for m, k in enumerate(cols):
        x[m, k] = 1.0
    W = oracle.dequantize(wq, s, b, 64, bits, "bfloat16")
    for y in (oracle.qmm_factored(x, wq, s, b, 64, bits, "bfloat16"),
              oracle.quantized_matmul(x, wq, s, b, 64, bits, "bfloat16")):
        for m, k in enumerate(cols):
            assert np.array_equal(y[m], W[:, k])


@pytest.mark.parametrize("bits,gs", [(4, 64), (8, 32), (4, 128)])
def test_qmm_factored_matches_brute_force(bits, gs):
    x, wq, s, b = _qmm_case(4, 7, 40, 512, gs, bits, dtype="float32")
    brute = oracle.quantized_matmul(x, wq, s, b, gs, bits, "float32", dequant_first=False)
    fact = oracle.qmm_factored(x, wq, s, b, gs, bits, "float32")
    err = np.abs(fact - brute).max() / np.abs(brute).max()
    assert err < 2e-6


def test_qmm_is_linear_and_not_transposed():
    x, wq, s, b = _qmm_case(5, 2, 24, 128, dtype="float32")
    y = oracle.quantized_matmul(x, wq, s, b, 64, 4, "float32", dequant_first=False)
    assert y.shape == (2, 24)
    y2 = oracle.quantized_matmul(3 * x[:1] + x[1:], wq, s, b, 64, 4, "float32", dequant_first=False)
    np.testing.assert_allclose(y2[0], 3 * y[0] + y[1], rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------------- A5


def test_rms_norm_eps_placement():
    """tests/test_scaffold.py:205-220: eps 0.25, weight 1.5 -- a misplaced eps
    moves results by percent. Constant row c: y = 1.5 c / sqrt(c^2 + 0.25)."""
    x = np.full((2, 32), 0.5, np.float32)
    x[1] = -2.0
    y = oracle.rms_norm(x, np.full(32, 1.5, np.float32), 0.25, "float32")
    assert y[0, 0] == pytest.approx(1.5 * 0.5 / math.sqrt(0.25 + 0.25), rel=1e-7)
    assert y[1, 0] == pytest.approx(1.5 * -2.0 / math.sqrt(4.0 + 0.25), rel=1e-7)


def test_rms_norm_two_roundings():
    """bf16: y = T(w * T(x * inv)); with w = 1.5 the inner rounding shows."""
    r = rng(6)
    x = oracle.round_to(r.normal(0, 1, (8, 64)), "bfloat16")
    w = np.full(64, 1.5, np.float32)
    y = oracle.rms_norm(x, w, 1e-6, "bfloat16")
    inv = 1 / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-6)
    inner = oracle.round_to(x * inv, "bfloat16")
    assert np.array_equal(y, oracle.round_to(1.5 * inner.astype(np.float64), "bfloat16"))


# ---------------------------------------------------------------------- A6


def test_rope_identity_at_position_zero():
    x = rng(7).normal(0, 1, (1, 2, 1, 16)).astype(np.float32)
    assert np.array_equal(oracle.rope(x, 16, False, 1e4, 1.0, 0, "float32"), x)


def test_rope_quarter_turn_sign_and_pairing():
    """theta_0 = (l + offset) * scale = pi/2 at l = 1: (a, b) -> (-b, a) on the
    non-traditional pair (0, D/2)."""
    x = np.zeros((1, 2, 4), np.float32)
    x[0, 1, 0], x[0, 1, 2] = 3.0, 5.0
    y = oracle.rope(x, 4, False, 1e4, math.pi / 2, 0, "float32")
    assert y[0, 1, 0] == pytest.approx(-5.0, abs=1e-6)
    assert y[0, 1, 2] == pytest.approx(3.0, abs=1e-6)


def test_rope_frequency_formula():
    """theta_j = pos * base^(-2j/dims): base 1e4, dims 4, j = 1 -> pos / 100."""
    x = np.zeros((1, 1, 4), np.float32)
    x[0, 0, 1] = 1.0
    y = oracle.rope(x, 4, False, 1e4, 1.0, 7, "float32")
    assert y[0, 0, 1] == pytest.approx(math.cos(0.07), abs=1e-7)
    assert y[0, 0, 3] == pytest.approx(math.sin(0.07), abs=1e-7)


def test_rope_preserves_pair_norms_and_tail():
    x = rng(8).normal(0, 1, (2, 3, 5, 16)).astype(np.float32)
    y = oracle.rope(x, 12, False, 1e6, 1.0, 3, "float32")
    assert np.array_equal(y[..., 12:], x[..., 12:])
    n0 = x[..., :6] ** 2 + x[..., 6:12] ** 2
    n1 = y[..., :6] ** 2 + y[..., 6:12] ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-5)


def test_rope_traditional_is_the_permuted_pairing():
    x = rng(9).normal(0, 1, (1, 4, 8)).astype(np.float32)
    perm = np.array([0, 2, 4, 6, 1, 3, 5, 7])   # interleaved -> split halves
    trad = oracle.rope(x, 8, True, 1e4, 1.0, 2, "float32")
    split = oracle.rope(x[..., perm], 8, False, 1e4, 1.0, 2, "float32")
    np.testing.assert_allclose(trad[..., perm], split, rtol=1e-6, atol=1e-7)


# ---------------------------------------------------------------------- A7


def _brute_sdpa(q, k, v, scale, causal):
    B, H, Lq, D = q.shape
    HK, Lk = k.shape[1], k.shape[2]
    out = np.zeros((B, H, Lq, D))
    for bb in range(B):
        for h in range(H):
            kv = h // (H // HK)
            for i in range(Lq):
                w = []
                for j in range(Lk):
                    if causal and j > i + Lk - Lq:
                        continue
                    w.append((j, math.exp(float(np.dot(q[bb, h, i], k[bb, kv, j])) * scale)))
                tot = sum(e for _, e in w)
                for j, e in w:
                    out[bb, h, i] += e / tot * v[bb, kv, j]
    return out


@pytest.mark.parametrize("causal,Lq,Lk", [(True, 5, 5), (True, 2, 6), (False, 3, 4)])
def test_sdpa_matches_brute_force_gqa(causal, Lq, Lk):
    r = rng(10)
    q = r.normal(0, 1, (1, 4, Lq, 8))
    k = r.normal(0, 1, (1, 2, Lk, 8))
    v = r.normal(0, 1, (1, 2, Lk, 8))
    got = oracle.sdpa(q, k, v, 0.35, causal, "float32")
    np.testing.assert_allclose(got, _brute_sdpa(q, k, v, 0.35, causal), rtol=1e-5, atol=1e-6)


def test_sdpa_invariants():
    r = rng(12)
    v = r.normal(0, 1, (1, 2, 6, 4))
    q = np.zeros((1, 4, 6, 4))
    k = r.normal(0, 1, (1, 2, 6, 4))
    o = oracle.sdpa(q, k, v, 1.0, True, "float32")
    # row 0 sees key 0 only; uniform scores average the visible prefix
    for h in range(4):
        np.testing.assert_allclose(o[0, h, 0], v[0, h // 2, 0], rtol=1e-6)
        for i in range(6):
            np.testing.assert_allclose(o[0, h, i], v[0, h // 2, : i + 1].mean(0), rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------------ A8-A10


def test_swiglu_and_gelu_closed_forms():
    g = np.array([0.0, 1.0, -2.0], np.float32)
    u = np.array([5.0, 2.0, 3.0], np.float32)
    y = oracle.swiglu(g, u, "float32")
    silu = [0.0, 1.0 / (1.0 + math.exp(-1.0)), -2.0 / (1.0 + math.exp(2.0))]
    np.testing.assert_allclose(y, [silu[i] * u[i] for i in range(3)], rtol=1e-6)
    got = oracle.gelu(np.array([0.0, 1.0, -1.0]))
    np.testing.assert_allclose(got, [0.0, 0.8413447460685429, -0.15865525393145707], rtol=1e-12)


def test_shortconv_known_answer_and_state():
    bx = np.array([[[1.0], [10.0], [100.0]]])
    c = np.ones_like(bx)
    w = np.array([[1.0, 2.0, 3.0]])
    out, st = oracle.shortconv(bx, c, w, None, "float32")
    assert out[0, :, 0].tolist() == [3.0, 32.0, 321.0]
    assert st[0, :, 0].tolist() == [10.0, 100.0]


def test_shortconv_chunked_equals_whole():
    r = rng(13)
    bx = r.normal(0, 1, (2, 7, 5))
    c = r.normal(0, 1, (2, 7, 5))
    w = r.normal(0, 1, (5, 3))
    whole, st_w = oracle.shortconv(bx, c, w, None, "float32")
    a, st = oracle.shortconv(bx[:, :3], c[:, :3], w, None, "float32")
    b_, st2 = oracle.shortconv(bx[:, 3:], c[:, 3:], w, st, "float32")
    np.testing.assert_allclose(np.concatenate([a, b_], 1), whole, rtol=1e-6)
    np.testing.assert_allclose(st2, st_w)


def test_split_gate_order_is_b_c_x():
    y = np.concatenate([np.full((1, 2), 2.0), np.full((1, 2), 3.0), np.full((1, 2), 5.0)], -1)
    c, bx = oracle.split_gate(y, "float32")
    assert c.tolist() == [[3.0, 3.0]] and bx.tolist() == [[10.0, 10.0]]


def test_tiny_mlp_bias_path():
    r = rng(14)
    x = r.normal(0, 1, (3, 8))
    w1 = r.normal(0, 0.02, (16, 8))
    y = oracle.tiny_mlp(x, w1, np.zeros(16), np.zeros((4, 16)), np.full(4, 0.25))
    assert (y == np.float32(0.25)).all()


def test_tiny_mlp_one_hot_closed_form():
    """W1 row j picks input k_j, W2 row n picks hidden unit j_n with weight c_n:
    y[m, n] = c_n * gelu(x[m, k_(j_n)] + b1[j_n]) + b2[n], with GELU from
    math.erf per scalar. A dropped b1, a GELU after the second linear or a
    transposed weight fails it."""
    import math

    r = rng(15)
    M, K, H, N = 5, 6, 7, 4
    x = r.normal(0, 1, (M, K))
    k_of = r.integers(0, K, H)
    j_of = r.integers(0, H, N)
    c = r.normal(0, 1, N)
    w1 = np.zeros((H, K))
    w1[np.arange(H), k_of] = 1.0
    w2 = np.zeros((N, H))
    w2[np.arange(N), j_of] = c
    b1 = r.normal(0, 1, H)
    b2 = r.normal(0, 1, N)
    y = oracle.tiny_mlp(x, w1, b1, w2, b2)
    for m in range(M):
        for n in range(N):
            hval = x[m, k_of[j_of[n]]] + b1[j_of[n]]
            want = c[n] * hval * (1.0 + math.erf(hval / math.sqrt(2.0))) / 2.0 + b2[n]
            assert abs(float(y[m, n]) - want) <= 1e-6 * max(1.0, abs(want)), (m, n)


def test_gelu_known_values():
    # exact GELU: x * Phi(x); Phi(1) = 0.8413447460685429
    g = oracle.gelu(np.array([0.0, 1.0, -1.0, 8.0, -8.0]))
    np.testing.assert_allclose(g, [0.0, 0.8413447460685429, -0.15865525393145707, 8.0, 0.0],
                               atol=1e-12)


# ---------------------------------------------------------------------- A12


def _tiny_cfg():
    from types import SimpleNamespace

    return SimpleNamespace(group_size=64, bits=4, rms_norm_eps=1e-6, num_attention_heads=4,
                           num_key_value_heads=2, head_dim=32, rope_theta=1e6)


def _tiny_layer(seed, hidden=128, inter=256, zero=()):
    cfg = _tiny_cfg()
    r = rng(seed)
    H, HK, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    shapes = {"q_proj": (H * D, hidden), "k_proj": (HK * D, hidden), "v_proj": (HK * D, hidden),
              "o_proj": (hidden, H * D), "gate_proj": (inter, hidden), "up_proj": (inter, hidden),
              "down_proj": (hidden, inter)}
    W = {}
    for name, (n, k) in shapes.items():
        wq, s, b = oracle.quantize_affine(r.normal(0, 0.05, (n, k)).astype(np.float32), 64, 4,
                                          "bfloat16")
        if name in zero:
            s, b = np.zeros_like(s), np.zeros_like(b)
        W[name] = (wq, s, b)
    for name, d in (("q_norm", D), ("k_norm", D), ("input_layernorm", hidden),
                    ("post_attention_layernorm", hidden)):
        W[name] = oracle.round_to(1 + 0.1 * r.normal(0, 1, d), "bfloat16")
    return cfg, W


def _caches(cfg, cap=16):
    kc = np.zeros((1, cfg.num_key_value_heads, cap, cfg.head_dim), np.float32)
    return kc, np.zeros_like(kc)


def test_layer_residual_structure():
    """o_proj and down_proj dequantizing to zero leave both residual adds
    with nothing to add: the layer is the identity, exactly (a missing or
    doubled residual, or a norm applied to the stream, fails)."""
    cfg, W = _tiny_layer(40, zero=("o_proj", "down_proj"))
    x = oracle.round_to(rng(41).normal(0, 1, (1, 5, 128)), "bfloat16")
    kc, vc = _caches(cfg)
    assert np.array_equal(oracle.qwen3_layer(x, W, cfg, 0, kc, vc), x)


def test_layer_decode_with_cache_equals_prefill_last_row():
    """A prefix through the layer fills the cache; the next token decoded at
    offset 5 against that cache matches the last row of a 6-token prefill
    (positions, rope offset, cache rows and the causal mask line up). The
    two take different qmm orderings (factored at M=1, dequantize-first at
    M=6), so agreement is to bf16 rounding."""
    cfg, W = _tiny_layer(42)
    seq = oracle.round_to(rng(43).normal(0, 1, (1, 6, 128)), "bfloat16")
    kc, vc = _caches(cfg)
    full = oracle.qwen3_layer(seq, W, cfg, 0, kc, vc)
    kc2, vc2 = _caches(cfg)
    oracle.qwen3_layer(seq[:, :5], W, cfg, 0, kc2, vc2)
    last = oracle.qwen3_layer(seq[:, 5:], W, cfg, 5, kc2, vc2)
    err = np.abs(last - full[:, 5:]).max() / np.abs(full[:, 5:]).max()
    assert err < 1e-2
    np.testing.assert_allclose(kc2[:, :, :6], kc[:, :, :6], rtol=0, atol=0.05)
    # a wrong offset (rope at position 0 instead of 5) is far outside that bar
    kc3, vc3 = _caches(cfg)
    oracle.qwen3_layer(seq[:, :5], W, cfg, 0, kc3, vc3)
    kc3[:, :, 5:] = 0
    wrong = oracle.qwen3_layer(seq[:, 5:], W, cfg, 0, kc3, vc3)
    assert np.abs(wrong - full[:, 5:]).max() / np.abs(full[:, 5:]).max() > 1e-2


def test_forward_embedding_gather_and_tied_head():
    """qwen3_forward with no layers: the embedding rows are the dequantized
    table rows and the logits are the factored qmm of the normed last row
    against the same table."""
    cfg = _tiny_cfg()
    r = rng(44)
    V, hidden = 96, 128
    emb = oracle.quantize_affine(r.normal(0, 0.05, (V, hidden)).astype(np.float32), 64, 4,
                                 "bfloat16")
    fn = oracle.round_to(1 + 0.1 * r.normal(0, 1, hidden), "bfloat16")
    ids = np.array([[3, 95, 0, 17]])
    logits = oracle.qwen3_forward(ids, [], emb, fn, cfg, 0, [], [])
    table = oracle.dequantize(*emb, 64, 4, "bfloat16")
    hn = oracle.rms_norm(table[ids[0, -1]][None, None], fn, cfg.rms_norm_eps, "bfloat16")
    want = oracle.round_to(hn.astype(np.float64) @ table.astype(np.float64).T, "bfloat16")
    assert logits.shape == (1, 1, V)
    err = np.abs(logits - want).max() / np.abs(want).max()
    assert err < 1e-2


# ---------------------------------------------------------------------- LFM2


def _tiny_lfm2(seed, hidden=128, inter=256, zero=()):
    from types import SimpleNamespace

    cfg = SimpleNamespace(group_size=64, bits=4, norm_eps=1e-5, num_attention_heads=4,
                          num_key_value_heads=2, head_dim=32, rope_theta=1e6)
    r = rng(seed)
    H, HK, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    shapes = {"in_proj": (3 * hidden, hidden), "out_proj": (hidden, H * D),
              "q_proj": (H * D, hidden), "k_proj": (HK * D, hidden), "v_proj": (HK * D, hidden),
              "w1": (inter, hidden), "w3": (inter, hidden), "w2": (hidden, inter)}
    W = {}
    for name, (n, k) in shapes.items():
        wq, s, b = oracle.quantize_affine(r.normal(0, 0.05, (n, k)).astype(np.float32), 64, 4,
                                          "bfloat16")
        if name in zero:
            s, b = np.zeros_like(s), np.zeros_like(b)
        W[name] = (wq, s, b)
    for name, d in (("q_layernorm", D), ("k_layernorm", D), ("operator_norm", hidden),
                    ("ffn_norm", hidden)):
        W[name] = oracle.round_to(1 + 0.1 * r.normal(0, 1, d), "bfloat16")
    W["conv"] = oracle.round_to(0.3 * r.normal(0, 1, (hidden, 3)), "bfloat16")
    return cfg, W


def test_lfm2_layers_residual_structure():
    """out_proj and w2 dequantizing to zero: both LFM2 layer kinds are the
    identity, exactly, and the conv layer still hands on its last two B*x
    rows as the state."""
    cfg, W = _tiny_lfm2(50, zero=("out_proj", "w2"))
    x = oracle.round_to(rng(51).normal(0, 1, (1, 5, 128)), "bfloat16")
    y, st = oracle.lfm2_conv_layer(x, W, cfg, None)
    assert np.array_equal(y, x)
    xn = oracle.rms_norm(x, W["operator_norm"], cfg.norm_eps, "bfloat16")
    _, bx = oracle.split_gate(oracle._qmm_auto(xn, W["in_proj"], 64, 4, "bfloat16"), "bfloat16")
    assert np.array_equal(st, bx[:, -2:])
    kc, vc = _caches(cfg)
    assert np.array_equal(oracle.lfm2_attn_layer(x, W, cfg, 0, kc, vc), x)


@pytest.mark.parametrize("split", [1, 2, 4])
def test_lfm2_conv_layer_chunks_equal_whole(split):
    """A 7-row sequence through the conv layer in two chunks, the state
    carried, is bit-identical to one pass (a state taken from B*x alone, or
    the wrong rows of it, fails when the first chunk is shorter than 2)."""
    cfg, W = _tiny_lfm2(52)
    x = oracle.round_to(rng(53).normal(0, 1, (1, 7, 128)), "bfloat16")
    whole, st_whole = oracle.lfm2_conv_layer(x, W, cfg, None)
    a, st = oracle.lfm2_conv_layer(x[:, :split], W, cfg, None)
    b, st2 = oracle.lfm2_conv_layer(x[:, split:], W, cfg, st)
    assert np.array_equal(np.concatenate([a, b], axis=1), whole)
    assert np.array_equal(st2, st_whole)


def test_lfm2_attn_decode_equals_prefill_last_row():
    """The LFM2 attention layer: a 5-token prefix fills the cache, the 6th
    token decoded at offset 5 matches the last row of a 6-token prefill; a
    wrong rope offset is far outside that bar."""
    cfg, W = _tiny_lfm2(54)
    seq = oracle.round_to(rng(55).normal(0, 1, (1, 6, 128)), "bfloat16")
    kc, vc = _caches(cfg)
    full = oracle.lfm2_attn_layer(seq, W, cfg, 0, kc, vc)
    kc2, vc2 = _caches(cfg)
    oracle.lfm2_attn_layer(seq[:, :5], W, cfg, 0, kc2, vc2)
    last = oracle.lfm2_attn_layer(seq[:, 5:], W, cfg, 5, kc2, vc2)
    assert np.abs(last - full[:, 5:]).max() / np.abs(full[:, 5:]).max() < 1e-2
    kc3, vc3 = _caches(cfg)
    oracle.lfm2_attn_layer(seq[:, :5], W, cfg, 0, kc3, vc3)
    wrong = oracle.lfm2_attn_layer(seq[:, 5:], W, cfg, 0, kc3, vc3)
    assert np.abs(wrong - full[:, 5:]).max() / np.abs(full[:, 5:]).max() > 1e-2


# ------------------------------------------------------- A6 head layout


def test_norm_rope_each_head_is_its_own_slice():
    """norm_rope(x [B, L, H*D]) at head h equals rms_norm then rope of the
    contiguous slice x[..., h*D:(h+1)*D] with positions along L: pins the
    reshape to [B, L, H, D] and the transpose to [B, H, L, D] (a [D, H] split or
    a missing transpose, which would rotate by head index, fails)."""
    r = rng(16)
    B, L, H, D = 2, 5, 3, 8
    x = oracle.round_to(r.normal(0, 1, (B, L, H * D)), "float32")
    w = oracle.round_to(r.normal(1, 0.1, D), "float32")
    out = oracle.norm_rope(x, w, 1e-6, H, D, 1e4, 3, "float32")
    assert out.shape == (B, H, L, D)
    for h in range(H):
        sl = x[:, :, h * D:(h + 1) * D]                       # [B, L, D]
        want = oracle.rope(oracle.rms_norm(sl, w, 1e-6, "float32"), D, False, 1e4, 1.0, 3,
                           "float32")
        np.testing.assert_array_equal(out[:, h], want)


def test_norm_rope_permuting_heads_permutes_outputs():
    r = rng(17)
    B, L, H, D = 1, 4, 4, 16
    x = oracle.round_to(r.normal(0, 1, (B, L, H, D)), "bfloat16")
    w = oracle.round_to(r.normal(1, 0.1, D), "bfloat16")
    perm = np.array([2, 0, 3, 1])
    a = oracle.norm_rope(x.reshape(B, L, H * D), w, 1e-6, H, D, 1e6, 0, "bfloat16")
    b = oracle.norm_rope(x[:, :, perm].reshape(B, L, H * D), w, 1e-6, H, D, 1e6, 0, "bfloat16")
    np.testing.assert_array_equal(b, a[:, perm])
    # one head: rms_norm over the row, then rope along the sequence
    one = oracle.norm_rope(x[:, :, 0], w, 1e-6, 1, D, 1e6, 2, "bfloat16")
    np.testing.assert_array_equal(
        one[:, 0], oracle.rope(oracle.rms_norm(x[:, :, 0], w, 1e-6, "bfloat16"), D, False, 1e6,
                               1.0, 2, "bfloat16"))


def test_layer_with_factored_projections_stays_within_the_bar():
    """The CPU baseline's layer (every projection through the C factored qmm)
    against the default oracle layer (dequantize-then-matmul at M > 8)."""
    cfg, W = _tiny_layer(31)
    x = oracle.round_to(rng(32).normal(0, 1, (1, 24, 128)), "bfloat16")
    kc = np.zeros((1, cfg.num_key_value_heads, 24, cfg.head_dim), np.float32)

    def proj(a, lin):
        return oracle.qmm_factored(a, *lin, cfg.group_size, cfg.bits, "bfloat16")

    a = oracle.qwen3_layer(x, W, cfg, 0, kc.copy(), kc.copy(), qmm=proj)
    b = oracle.qwen3_layer(x, W, cfg, 0, kc.copy(), kc.copy())
    assert np.abs(a - b).max() <= 1e-2 * np.abs(b).max()


@pytest.mark.parametrize("kind", ["conv", "attn"])
@pytest.mark.parametrize("rows", [9, 16, 31])
def test_lfm2_layer_window_equals_the_whole_layer(kind, rows):
    """oracle.lfm2_layer_window (the teacher-forced window of the config-5 GPU
    test) gives the whole layer's last rows bit for bit: the conv window's two
    context rows and the attention window's key/value prefix carry exactly
    what those rows read (a window without the context rows, or without the
    prefix, fails)."""
    cfg, W = _tiny_lfm2(60)
    L = 40
    x = oracle.round_to(rng(61).normal(0, 1, (1, L, 128)), "bfloat16")
    if kind == "conv":
        whole, _ = oracle.lfm2_conv_layer(x, W, cfg, None)
    else:
        kc, vc = _caches(cfg, L)
        whole = oracle.lfm2_attn_layer(x, W, cfg, 0, kc, vc)
    got = oracle.lfm2_layer_window(x, W, cfg, kind, rows)
    assert got.shape == (1, rows, 128)
    assert np.array_equal(got, whole[:, L - rows:])
    # the window alone (no context rows / no key prefix) is a different answer
    if kind == "conv":
        alone, _ = oracle.lfm2_conv_layer(x[:, L - rows:], W, cfg, None)
    else:
        kc, vc = _caches(cfg, L)
        alone = oracle.lfm2_attn_layer(x[:, L - rows:], W, cfg, 0, kc, vc)
    assert not np.array_equal(alone, whole[:, L - rows:])
    with pytest.raises(ValueError):  # projections of <= 8 rows route to the qmv form
        oracle.lfm2_layer_window(x, W, cfg, kind, 8)
