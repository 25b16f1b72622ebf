"""LFM2 hybrid parity (benchmark config 5): the gated short-conv and attention
layers, 4- and 8-bit, with the region wrappers installed vs the original op
streams, and both against the CPU oracle compositions (oracle.lfm2_conv_layer /
lfm2_attn_layer, following the reference's patch/wrappers.py op streams).

Bars: the region-wrapped layer equals the original op stream bit for bit
(every fused epilogue keeps the unfused ops' roundings); against the oracle,
max-abs-normalised error <= 1e-2 (bf16) per layer output, conv state and
logits; chunked prefill (mlx-lm's 2048-token pieces, the conv state and KV
cache carried) equals one pass over the whole prompt bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import to_np, to_torch

torch = pytest.importorskip("torch")


def _lin(m):
    return (m.weight.cpu().numpy().view(np.uint32), m.scales.float().cpu().numpy(),
            m.biases.float().cpu().numpy())


def export_layer(layer) -> dict:
    """The weights of an LFM2 layer (either kind) in the oracle's dict form."""
    layer = layer.wrapped if hasattr(layer, "wrapped") else layer
    W = {"operator_norm": to_np(layer.operator_norm.weight), "ffn_norm": to_np(layer.ffn_norm.weight)}
    ff = layer.feed_forward
    W.update(w1=_lin(ff.w1), w3=_lin(ff.w3), w2=_lin(ff.w2))
    if hasattr(layer, "conv"):
        c = layer.conv
        D = c.out_proj.weight.shape[0]
        W.update(in_proj=_lin(c.in_proj), out_proj=_lin(c.out_proj),
                 conv=to_np(c.conv.weight).reshape(D, 3))
    else:
        a = layer.self_attn
        W.update(q_proj=_lin(a.q_proj), k_proj=_lin(a.k_proj), v_proj=_lin(a.v_proj),
                 out_proj=_lin(a.out_proj), q_layernorm=to_np(a.q_layernorm.weight),
                 k_layernorm=to_np(a.k_layernorm.weight))
    return W


def _close(got, want, tol=1e-2):
    err = np.abs(got.astype(np.float64) - want).max() / max(np.abs(want).max(), 1e-30)
    assert err <= tol, f"max-abs-normalised error {err:.3e} > {tol}"
    return err


def _x(seed, L, hidden):
    r = np.random.Generator(np.random.PCG64(seed))
    return oracle.round_to(r.normal(0, 1, (1, L, hidden)), "bfloat16")


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [4, 8])
def test_lfm2_conv_layer(bits):
    """A conv layer at L=256 from a fresh state, then a 64-row chunk carrying
    the state: regions == original ops bit for bit, and <= 1e-2 of the oracle
    (outputs and the carried state)."""
    from workloads import lfm2

    cfg = lfm2.Lfm2Config(bits=bits)
    model = lfm2.build(cfg, seed=5, num_layers=1, layer_types=("conv",))
    layer = model.model.layers[0]
    x1, x2 = _x(6, 256, cfg.hidden_size), _x(7, 64, cfg.hidden_size)

    def run(mod):
        cache = lfm2.ConvCache()
        y1 = mod(to_torch(x1, "bfloat16"), cache)
        s1 = cache.state
        y2 = mod(to_torch(x2, "bfloat16"), cache)
        return y1, s1, y2, cache.state

    orig = run(layer)
    reg = run(lfm2.Lfm2ConvRegions(layer, lfm2.layer_specs(cfg)))
    torch.cuda.synchronize()
    for a, b in zip(orig, reg):
        assert torch.equal(a, b), "region splice changed the conv layer's bits"

    W = export_layer(layer)
    want1, st1 = oracle.lfm2_conv_layer(x1, W, cfg, None)
    want2, st2 = oracle.lfm2_conv_layer(x2, W, cfg, to_np(reg[1]))
    e1 = _close(to_np(reg[0]), want1)
    _close(to_np(reg[1]), st1)
    e2 = _close(to_np(reg[2]), want2)
    _close(to_np(reg[3]), st2)
    print(f"\nlfm2 conv layer {bits}-bit: max-abs-normalised error {e1:.3e} (L=256), "
          f"{e2:.3e} (chunk with state)")


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [4, 8])
def test_lfm2_attn_layer(bits):
    """An attention layer (D=64, 32/8 heads): prefill L=256, then one decode
    token at offset 256 through the same KV cache."""
    from workloads import lfm2

    cfg = lfm2.Lfm2Config(bits=bits)
    model = lfm2.build(cfg, seed=8, num_layers=1, layer_types=("attn",))
    layer = model.model.layers[0]
    x1, x2 = _x(9, 256, cfg.hidden_size), _x(10, 1, cfg.hidden_size)
    cap = 512

    def run(mod):
        cache = lfm2.KVCache(cfg.num_key_value_heads, cfg.head_dim, cap, "cuda")
        y1 = mod(to_torch(x1, "bfloat16"), cache)
        cache.offset = 256
        y2 = mod(to_torch(x2, "bfloat16"), cache)
        return y1, y2, cache

    o1, o2, oc = run(layer)
    r1, r2, rc = run(lfm2.Lfm2AttnRegions(layer, lfm2.layer_specs(cfg)))
    torch.cuda.synchronize()
    assert torch.equal(o1, r1) and torch.equal(o2, r2), "region splice changed the layer's bits"
    assert torch.equal(oc.keys, rc.keys) and torch.equal(oc.values, rc.values)

    W = export_layer(layer)
    kc = np.zeros((1, cfg.num_key_value_heads, cap, cfg.head_dim), np.float32)
    vc = np.zeros_like(kc)
    e1 = _close(to_np(r1), oracle.lfm2_attn_layer(x1, W, cfg, 0, kc, vc))
    e2 = _close(to_np(r2), oracle.lfm2_attn_layer(x2, W, cfg, 256, kc, vc))
    _close(to_np(rc.keys)[:, :, :257], kc[:, :, :257])
    print(f"\nlfm2 attention layer {bits}-bit: max-abs-normalised error {e1:.3e} (prefill), "
          f"{e2:.3e} (decode)")


def _hidden_states(model, ids, caches):
    inner = model.model
    hs = [inner.embed_tokens(ids)]
    for layer, c in zip(inner.layers, caches):
        hs.append(layer(hs[-1], c))
    for c in caches:
        c.offset += ids.shape[1]
    logits = inner.embed_tokens.as_linear(inner.embedding_norm(hs[-1][:, -1:, :]))
    return hs, logits


WINDOW = 128  # teacher-forced rows per layer: the last WINDOW positions of the prompt


def _teacher_forced_window(layer, x_in, cfg):
    """The oracle's output over the last WINDOW rows of one layer given the
    GPU's own whole input to it (oracle.lfm2_layer_window)."""
    base = layer.wrapped if hasattr(layer, "wrapped") else layer
    kind = "conv" if hasattr(base, "conv") else "attn"
    return oracle.lfm2_layer_window(x_in, export_layer(layer), cfg, kind, WINDOW)


@pytest.mark.gpu
@pytest.mark.timeout(900)
@pytest.mark.parametrize("bits", [4, 8])
def test_lfm2_model_config5_prefill(bits):
    """Config 5: 16 layers (conv at 0,1,3,4,6,7,9,11,13,15; attention at
    2,5,8,10,12,14), 4- and 8-bit, tied V=65536, a 2048-token prefill, then one
    greedy decode step through the carried KV caches and conv states.

    (a) the region-installed model equals the original op streams bit for
        bit, layer by layer and at the logits;
    (b) teacher-forced, every one of the 16 layers: the oracle layer on the
        GPU's own input to it, <= 1e-2 over the last 128 positions (conv
        layer 0 and attention layer 2 also over all 2048);
    (c) the final norm + tied lm_head on the GPU's last hidden state <= 1e-2,
        and the greedy token equal to the oracle's;
    (d) the decode step: every layer teacher-forced against the oracle layer
        on the GPU's decode input and the GPU's prefill state (its KV cache or
        conv state), <= 1e-2; the final norm + lm_head on the GPU's decode
        hidden state <= 1e-2 with the same greedy token; and the oracle's own
        chain of all 16 layers from the decoded token's embedding, over those
        states, gives the same token wherever its top-2 margin exceeds twice
        its drift from the GPU's logits.
    """
    from autotuner_runtime import ops
    from workloads import lfm2, qwen3

    cfg = lfm2.Lfm2Config(bits=bits)
    model = lfm2.build(cfg, seed=0)
    L = 2048
    ids = qwen3.tokens(11, L, cfg.vocab_size)
    hs_o, lg_o = _hidden_states(model, ids, model.make_cache(L + 1))
    hs_o = [to_np(h) for h in hs_o]
    lfm2.install_regions(model)
    caches = model.make_cache(L + 1)
    hs_r, lg_r = _hidden_states(model, ids, caches)
    torch.cuda.synchronize()
    for i, h in enumerate(hs_r):
        assert np.array_equal(to_np(h), hs_o[i]), f"layer {i}: regions changed the bits"
    assert torch.equal(lg_o, lg_r)
    hs = [to_np(h) for h in hs_r]

    inner = model.model
    layers = list(inner.layers)
    W0, W2 = export_layer(layers[0]), export_layer(layers[2])
    want0, _ = oracle.lfm2_conv_layer(hs[0], W0, cfg, None)
    e0 = _close(hs[1], want0)
    kc = np.zeros((1, cfg.num_key_value_heads, L, cfg.head_dim), np.float32)
    e2 = _close(hs[3], oracle.lfm2_attn_layer(hs[2], W2, cfg, 0, kc, np.zeros_like(kc)))
    errs = []
    for i, layer in enumerate(layers):
        want = _teacher_forced_window(layer, hs[i], cfg)
        errs.append(_close(hs[i + 1][:, L - WINDOW:], want))

    emb = _lin(inner.embed_tokens)
    hn = oracle.rms_norm(hs[-1][:, -1:], to_np(inner.embedding_norm.weight), cfg.norm_eps,
                         "bfloat16")
    want = oracle.qmm_factored(hn, *emb, cfg.group_size, cfg.bits, "bfloat16").reshape(-1)
    got = to_np(lg_r).reshape(-1)
    el = _close(got, want)
    tok = int(ops.argmax(lg_r.reshape(1, -1)).item())
    top2 = np.sort(want)[-2:]
    margin, abs_err = float(top2[1] - top2[0]), float(np.abs(got - want).max())
    print(f"\nconfig5 {bits}-bit prefill {L}: conv layer 0 {e0:.3e}, attention layer 2 "
          f"{e2:.3e} (whole prompt); every layer over the last {WINDOW} rows "
          f"max {max(errs):.3e}; logits {el:.3e} (top-2 margin {margin:.3e}, max abs err "
          f"{abs_err:.3e}), greedy token gpu {tok} oracle {int(np.argmax(want))}")
    assert tok == int(np.argmax(want)), "greedy token differs from the oracle's"

    # (d) one decode step through the carried states
    states = []
    for layer, c in zip(layers, caches):
        base = layer.wrapped if hasattr(layer, "wrapped") else layer
        if hasattr(base, "conv"):
            states.append(to_np(c.state).copy())
        else:
            states.append((to_np(c.keys).copy(), to_np(c.values).copy()))
    nxt = torch.tensor([[tok]], dtype=torch.int64, device="cuda")
    hd, lg_d = _hidden_states(model, nxt, caches)
    torch.cuda.synchronize()
    hd = [to_np(h) for h in hd]
    assert all(c.offset == L + 1 for c in caches)

    def oracle_layer(i, x):
        W = export_layer(layers[i])
        st = states[i]
        if isinstance(st, tuple):
            kc, vc = st[0].copy(), st[1].copy()
            return oracle.lfm2_attn_layer(x, W, cfg, L, kc, vc)
        return oracle.lfm2_conv_layer(x, W, cfg, st)[0]

    derrs = [_close(hd[i + 1], oracle_layer(i, hd[i])) for i in range(len(layers))]
    # the final norm + tied lm_head on the GPU's decode hidden state
    norm_w = to_np(inner.embedding_norm.weight)

    def head(x):
        hn = oracle.rms_norm(x, norm_w, cfg.norm_eps, "bfloat16")
        return oracle.qmm_factored(hn, *emb, cfg.group_size, cfg.bits, "bfloat16").reshape(-1)

    got_d = to_np(lg_d).reshape(-1)
    want_d = head(hd[-1])
    ed = _close(got_d, want_d)
    tok_d = int(ops.argmax(lg_d.reshape(1, -1)).item())
    assert tok_d == int(np.argmax(want_d)), "decode greedy token differs from the oracle's"
    # the oracle's own 16-layer chain from the embedding of the decoded token
    # (not teacher-forced: bf16 roundings drift apart layer by layer, so its
    # logits are reported, and its token must agree wherever its top-2 margin
    # exceeds the drift)
    xo = oracle.dequantize(*emb, cfg.group_size, cfg.bits, "bfloat16")[[tok]][None]
    assert np.array_equal(hd[0], xo)
    for i in range(len(layers)):
        xo = oracle_layer(i, xo)
    chain = head(xo)
    drift = float(np.abs(got_d - chain).max())
    top2 = np.sort(chain)[-2:]
    print(f"config5 {bits}-bit decode at {L}: layers teacher-forced max {max(derrs):.3e}, logits "
          f"{ed:.3e}, greedy token gpu {tok_d} oracle {int(np.argmax(want_d))}; oracle chain: "
          f"token {int(np.argmax(chain))}, logits drift {drift:.3e}, top-2 margin "
          f"{float(top2[1] - top2[0]):.3e}")
    if float(top2[1] - top2[0]) > 2 * drift:
        assert tok_d == int(np.argmax(chain)), "decode token differs from the oracle chain's"


@pytest.mark.gpu
@pytest.mark.timeout(600)
def test_lfm2_chunked_prefill_equals_whole():
    """mlx-lm's chunked prefill: 2560 tokens as pieces of 2048 and 512, the
    conv states and KV caches carried, gives the logits of one 2560-token
    pass bit for bit (8-bit weights, conv and attention layers)."""
    from workloads import lfm2, qwen3

    cfg = lfm2.Lfm2Config(bits=8)
    model = lfm2.build(cfg, seed=12, layer_types=("conv", "attn", "conv", "attn"))
    lfm2.install_regions(model)
    ids = qwen3.tokens(13, 2560, cfg.vocab_size)
    whole = model.forward(ids, model.make_cache(2560))
    caches = model.make_cache(2560)
    chunked = model.prefill(ids, caches, chunk=2048)
    torch.cuda.synchronize()
    assert all(c.offset == 2560 for c in caches)
    assert torch.equal(whole, chunked)
