"""Model-level parity: the Qwen3-4B-shaped layer (config 3) and model
(config 4), region wrappers installed vs the original op sequence, and both
against the CPU oracle composition (oracle.qwen3_layer / qwen3_forward).

Bars: the region-wrapped layer equals the original op sequence bit for bit
(the fused epilogues keep every rounding of the unfused ops); against the
oracle, max-abs-normalised error <= 1e-2 (bf16) per layer output and for the
final logits, and greedy tokens identical to the oracle's for the config-4
prefill and decode step (the top-2 margin is printed).
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import to_np, to_torch

torch = pytest.importorskip("torch")


def test_torch_quantizer_matches_oracle_quantizer():
    """The set-up quantizer (workloads.quantize, torch) and the oracle's produce
    identical packed words, scales and biases (CPU)."""
    from workloads.quantize import quantize_affine

    r = np.random.Generator(np.random.PCG64(3))
    for bits, gs in ((4, 64), (8, 32)):
        w = r.normal(0, 0.02, (48, 512)).astype(np.float32)
        wq, s, b = quantize_affine(torch.from_numpy(w), gs, bits, torch.bfloat16)
        owq, os_, ob = oracle.quantize_affine(w, gs, bits, "bfloat16")
        assert np.array_equal(wq.numpy().view(np.uint32), owq)
        assert np.array_equal(s.float().numpy(), os_) and np.array_equal(b.float().numpy(), ob)


def _lin(m):
    return (m.weight.cpu().numpy().view(np.uint32), m.scales.float().cpu().numpy(),
            m.biases.float().cpu().numpy())


def export_layer(layer) -> dict:
    a, m = layer.self_attn, layer.mlp
    return {
        "q_proj": _lin(a.q_proj), "k_proj": _lin(a.k_proj), "v_proj": _lin(a.v_proj),
        "o_proj": _lin(a.o_proj), "gate_proj": _lin(m.gate_proj), "up_proj": _lin(m.up_proj),
        "down_proj": _lin(m.down_proj),
        "q_norm": to_np(a.q_norm.weight), "k_norm": to_np(a.k_norm.weight),
        "input_layernorm": to_np(layer.input_layernorm.weight),
        "post_attention_layernorm": to_np(layer.post_attention_layernorm.weight),
    }


def _close(got, want, tol=1e-2):
    err = np.abs(got.astype(np.float64) - want).max() / max(np.abs(want).max(), 1e-30)
    assert err <= tol, f"max-abs-normalised error {err:.3e} > {tol}"
    return err


@pytest.mark.gpu
@pytest.mark.parametrize("L,offset", [(128, 0), (1, 128)])
def test_qwen3_layer_config3(L, offset, monkeypatch):
    from workloads import qwen3

    fused = []  # the region model's fused q/k/v + prologue: taken (True) or declined
    real = qwen3.ops.qkv_norm_rope

    def counting(*a, **k):
        out = real(*a, **k)
        fused.append(out is not None)
        return out

    monkeypatch.setattr(qwen3.ops, "qkv_norm_rope", counting)

    cfg = qwen3.Qwen3Config()
    model = qwen3.build(cfg, seed=3, num_layers=1)
    layer = model.model.layers[0]
    r = np.random.Generator(np.random.PCG64(4))
    x = oracle.round_to(r.normal(0, 1, (1, L, cfg.hidden_size)), "bfloat16")
    prefix = oracle.round_to(r.normal(0, 1, (1, offset, cfg.hidden_size)), "bfloat16") if offset else None

    def run(mod):
        cache = qwen3.KVCache(cfg.num_key_value_heads, cfg.head_dim, 256, "cuda")
        if offset:  # fill the cache with a prefix through the same layer
            mod(to_torch(prefix, "bfloat16"), cache)
            cache.offset = offset
        return mod(to_torch(x, "bfloat16"), cache), cache

    y_orig, c_orig = run(layer)
    wrapped = qwen3.Qwen3LayerRegions(layer, qwen3.layer_specs(cfg))
    y_reg, c_reg = run(wrapped)
    torch.cuda.synchronize()
    assert torch.equal(y_orig, y_reg), "region splice changed the layer output bits"
    assert torch.equal(c_orig.keys, c_reg.keys) and torch.equal(c_orig.values, c_reg.values)
    # prefill sizes take the fused launch, the decode step (M = 1) the two launches
    assert fused == ([True] if not offset else [True, False]), fused

    W = export_layer(layer)
    kc = np.zeros((1, cfg.num_key_value_heads, 256, cfg.head_dim), np.float32)
    vc = np.zeros_like(kc)
    if offset:
        oracle.qwen3_layer(prefix, W, cfg, 0, kc, vc)
    want = oracle.qwen3_layer(x, W, cfg, offset, kc, vc)
    err = _close(to_np(y_reg), want)
    print(f"\nconfig3 L={L} offset={offset}: max-abs-normalised error {err:.3e}")
    _close(to_np(c_reg.keys)[:, :, :offset + L], kc[:, :, :offset + L])


@pytest.mark.gpu
def test_qwen3_linked_layers_equal_unlinked_and_original():
    """install_regions links neighbouring layers: layer i's down_proj cut also
    normalizes layer i+1's input (NormHandoff). A 3-layer model's prefill
    (K parts at M = 128) and decode step (M = 1) give the original ops'
    logits bit for bit with and without the links, and every link is used."""
    from workloads import qwen3

    cfg = qwen3.Qwen3Config()
    ids = qwen3.tokens(5, 128, cfg.vocab_size)
    used = []
    put = qwen3.NormHandoff.put

    def counting_put(self, h, hn):
        used.append(h.shape[1])
        put(self, h, hn)

    def run(link):
        model = qwen3.build(cfg, seed=6, num_layers=3)
        if link is not None:
            qwen3.install_regions(model, link_layers=link)
        caches = model.make_cache(256)
        a = model(ids, caches)
        b = model(ids[:, :1], caches)
        torch.cuda.synchronize()
        return a, b

    want = run(None)
    assert all(torch.equal(g, w) for g, w in zip(run(False), want))
    qwen3.NormHandoff.put = counting_put
    try:
        got = run(True)
    finally:
        qwen3.NormHandoff.put = put
    assert all(torch.equal(g, w) for g, w in zip(got, want))
    assert used == [128, 128, 1, 1], used


@pytest.mark.gpu
@pytest.mark.timeout(900)
def test_qwen3_model_config4_prefill_and_decode():
    """36 layers + tied quantized embedding/lm_head (V = 151936), prefill of 128
    seeded token ids, then one greedy decode step with the KV cache.

    (a) every layer, teacher-forced: the oracle layer on the GPU's own layer
        input vs the GPU layer output, <= 1e-2 max-abs-normalised;
    (b) the embedding gather bit-exact and the final norm + lm_head on the
        GPU's last hidden state <= 1e-2;
    (c) free-running: the oracle model from the same token ids (its decode
        step fed the GPU's prefill token); the logit drift (1-ulp bf16
        rounding flips compound through 36 random-weight layers) stays under
        0.1 and both greedy tokens equal the oracle's.
    """
    from autotuner_runtime import ops
    from workloads import qwen3

    cfg = qwen3.Qwen3Config()
    model = qwen3.build(cfg, seed=0)
    qwen3.install_regions(model)
    ids = qwen3.tokens(1, 128, cfg.vocab_size)
    cap = 256
    caches = model.make_cache(cap)
    inner = model.model

    def run(step_ids, offset):
        hs = [inner.embed_tokens(step_ids)]
        for layer, c in zip(inner.layers, caches):
            c.offset = offset
            hs.append(layer(hs[-1], c))
        for c in caches:
            c.offset = offset + step_ids.shape[1]
        logits = inner.embed_tokens.as_linear(inner.norm(hs[-1][:, -1:, :]))
        return [to_np(h) for h in hs], logits

    hs0, logits0 = run(ids, 0)
    tok0 = int(ops.argmax(logits0.reshape(1, -1)).item())
    assert tok0 == int(torch.argmax(logits0.float().reshape(-1)))
    hs1, logits1 = run(torch.tensor([[tok0]], device="cuda"), 128)
    tok1 = int(ops.argmax(logits1.reshape(1, -1)).item())

    layers = [export_layer(l.wrapped if hasattr(l, "wrapped") else l) for l in inner.layers]
    emb = _lin(inner.embed_tokens)
    fn = to_np(inner.norm.weight)
    W_emb = oracle.dequantize(*emb, cfg.group_size, cfg.bits, "bfloat16")
    assert np.array_equal(hs0[0][0], W_emb[ids.cpu().numpy()[0]])

    # (a) teacher-forced layers, prefill then decode (caches filled from the GPU inputs)
    kcs = [np.zeros((1, cfg.num_key_value_heads, cap, cfg.head_dim), np.float32) for _ in layers]
    vcs = [np.zeros_like(k) for k in kcs]
    worst = 0.0
    for hs, offset in ((hs0, 0), (hs1, 128)):
        for i, W in enumerate(layers):
            want = oracle.qwen3_layer(hs[i], W, cfg, offset, kcs[i], vcs[i])
            worst = max(worst, _close(hs[i + 1], want))
    print(f"\nconfig4 teacher-forced layers: worst max-abs-normalised error {worst:.3e}")
    # (b) lm_head on the GPU's final hidden state
    for hs, got in ((hs0, logits0), (hs1, logits1)):
        hn = oracle.rms_norm(hs[-1][:, -1:], fn, cfg.rms_norm_eps, "bfloat16")
        _close(to_np(got), oracle.qmm_factored(hn, *emb, cfg.group_size, cfg.bits, "bfloat16"))

    # (c) free-running oracle; its decode step takes the GPU's greedy token,
    # so both decode steps see the same input
    kcs = [np.zeros_like(k) for k in kcs]
    vcs = [np.zeros_like(k) for k in kcs]
    want0 = oracle.qwen3_forward(ids.cpu().numpy(), layers, emb, fn, cfg, 0, kcs, vcs)
    want1 = oracle.qwen3_forward(np.array([[tok0]]), layers, emb, fn, cfg, 128, kcs, vcs)
    for got, want, tok, name in ((logits0, want0, tok0, "prefill"), (logits1, want1, tok1, "decode")):
        g = to_np(got).reshape(-1)
        w = want.reshape(-1)
        err = np.abs(g - w).max() / np.abs(w).max()
        top2 = np.sort(w)[-2:]
        margin = float(top2[1] - top2[0])
        abs_err = float(np.abs(g - w).max())
        print(f"config4 {name} free-running: logits max-abs-normalised drift {err:.3e} "
              f"(max abs {abs_err:.3e}), oracle top-2 margin {margin:.3e}, "
              f"greedy token gpu {tok} oracle {int(np.argmax(w))}")
        # Free-running drift is 1-ulp bf16 rounding differences compounded
        # through 36 random-weight layers (each layer is held to 1e-2 in (a));
        # measured 4.5e-2 (prefill) and 4.7e-2 (decode). The bar is about
        # twice that: a real defect (a dropped term, a wrong rounding point)
        # drifts by O(1).
        assert err < 0.1, f"{name}: logits drift {err:.3e} is beyond rounding compounding"
        assert tok == int(np.argmax(w)), f"{name}: greedy token differs from the oracle's"


def ops_argmax(logits) -> int:
    from autotuner_runtime import ops

    return int(ops.argmax(logits.reshape(1, -1)).item())
