"""Write the committed golden fixtures (tests/golden/*.npz) from the CPU oracle.

The reference stores no arithmetic vectors for this path: its parity tests
compare live against MLX on an Apple GPU (tests/test_stitch.py,
tests/test_scaffold.py), and MLX is not installable here. These fixtures are
this build's own: small seeded inputs and the oracle's outputs, written once
and committed, so that

* a later change to the oracle that moves any output bit is caught
  (tests/test_golden.py recomputes every case and requires identical bits);
* the GPU parity tests have fixed vectors that do not depend on the oracle
  running on the GPU box.

Each case is one .npz (no pickles) holding inputs and expected outputs as
float32 (bf16/fp16 values are exact in float32), uint32 for packed words and
int32 for indices, plus a small JSON ``meta`` string with the scalars.

    python tests/golden/make_golden.py       # rewrites every fixture
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402  (test infrastructure; the product never imports it)


def _rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def _quant(r, n, k, gs, bits, dtype, spread=0.02):
    w = r.normal(0, spread, (n, k)).astype(np.float32)
    return oracle.quantize_affine(w, gs, bits, dtype)


def case_dequant(bits, gs, dtype, n, k, seed):
    r = _rng(seed)
    wq, s, b = _quant(r, n, k, gs, bits, dtype)
    out = oracle.dequantize(wq, s, b, gs, bits, dtype)
    meta = {"op": "dequant", "bits": bits, "group_size": gs, "dtype": dtype}
    return meta, {"w": wq, "scales": s, "biases": b}, {"out": out}


def case_qmm(bits, gs, dtype, m, n, k, seed):
    r = _rng(seed)
    wq, s, b = _quant(r, n, k, gs, bits, dtype)
    x = oracle.round_to(r.normal(0, 1, (m, k)), dtype)
    y = oracle.quantized_matmul(x, wq, s, b, gs, bits, dtype)
    meta = {"op": "qmm", "bits": bits, "group_size": gs, "dtype": dtype}
    return meta, {"x": x, "w": wq, "scales": s, "biases": b}, {"y": y}


def case_rms(dtype, m, d, eps, seed):
    r = _rng(seed)
    x = oracle.round_to(r.normal(0, 1, (m, d)), dtype)
    w = oracle.round_to(1 + 0.1 * r.normal(0, 1, d), dtype)
    return ({"op": "rms_norm", "eps": eps, "dtype": dtype}, {"x": x, "weight": w},
            {"y": oracle.rms_norm(x, w, eps, dtype)})


def case_norm_rope(dtype, L, H, D, offset, seed):
    r = _rng(seed)
    x = oracle.round_to(r.normal(0, 1, (1, L, H * D)), dtype)
    w = oracle.round_to(1 + 0.1 * r.normal(0, 1, D), dtype)
    meta = {"op": "norm_rope", "eps": 1e-6, "heads": H, "dims": D, "base": 1e6,
            "offset": offset, "dtype": dtype}
    y = oracle.norm_rope(x, w, 1e-6, H, D, 1e6, offset, dtype)
    return meta, {"x": x, "weight": w}, {"y": y}


def case_sdpa(dtype, H, HK, L, D, seed):
    r = _rng(seed)
    q = oracle.round_to(r.normal(0, 1, (1, H, L, D)), dtype)
    k = oracle.round_to(r.normal(0, 1, (1, HK, L, D)), dtype)
    v = oracle.round_to(r.normal(0, 1, (1, HK, L, D)), dtype)
    scale = float(D) ** -0.5
    o = oracle.sdpa(q, k, v, scale, True, dtype)
    return {"op": "sdpa", "scale": scale, "causal": True, "dtype": dtype}, \
        {"q": q, "k": k, "v": v}, {"o": o}


def case_swiglu(dtype, m, n, seed):
    r = _rng(seed)
    g = oracle.round_to(r.normal(0, 2, (m, n)), dtype)
    u = oracle.round_to(r.normal(0, 1, (m, n)), dtype)
    return {"op": "swiglu", "dtype": dtype}, {"g": g, "u": u}, {"y": oracle.swiglu(g, u, dtype)}


def case_shortconv(dtype, L, D, with_state, seed):
    r = _rng(seed)
    bx = oracle.round_to(r.normal(0, 1, (1, L, D)), dtype)
    c = oracle.round_to(r.normal(0, 1, (1, L, D)), dtype)
    w = oracle.round_to(r.normal(0, 0.5, (D, 3)), dtype)
    st = oracle.round_to(r.normal(0, 1, (1, 2, D)), dtype) if with_state else None
    out, new_state = oracle.shortconv(bx, c, w, st, dtype)
    ins = {"bx": bx, "c": c, "w": w}
    if st is not None:
        ins["state"] = st
    return {"op": "shortconv", "dtype": dtype}, ins, {"out": out, "state_out": new_state}


def case_tiny_mlp(m, d, h, seed):
    r = _rng(seed)
    x = r.normal(0, 1, (m, d)).astype(np.float32)
    w1 = r.normal(0, 0.02, (h, d)).astype(np.float32)
    b1 = r.normal(0, 0.1, h).astype(np.float32)
    w2 = r.normal(0, 0.02, (d, h)).astype(np.float32)
    b2 = r.normal(0, 0.1, d).astype(np.float32)
    y = oracle.tiny_mlp(x, w1, b1, w2, b2)
    return {"op": "tiny_mlp", "dtype": "float32"}, \
        {"x": x, "w1": w1, "b1": b1, "w2": w2, "b2": b2}, {"y": y}


def case_argmax(n, seed):
    r = _rng(seed)
    x = oracle.round_to(r.normal(0, 1, (3, n)), "bfloat16")
    x[1, 17] = x[1, 400] = x[1].max() + 1.0      # a tie: the lower index wins
    return {"op": "argmax", "dtype": "bfloat16"}, {"x": x}, \
        {"idx": np.argmax(x, axis=-1).astype(np.int32)}


CASES = {
    "dequant_b4_g64_bf16": lambda: case_dequant(4, 64, "bfloat16", 24, 256, 101),
    "dequant_b8_g32_fp16": lambda: case_dequant(8, 32, "float16", 16, 128, 102),
    "dequant_b4_g128_fp32": lambda: case_dequant(4, 128, "float32", 8, 256, 103),
    "qmm_b4_g64_bf16_m1": lambda: case_qmm(4, 64, "bfloat16", 1, 64, 512, 111),
    "qmm_b4_g64_bf16_m5": lambda: case_qmm(4, 64, "bfloat16", 5, 64, 512, 112),
    "qmm_b8_g64_fp16_m3": lambda: case_qmm(8, 64, "float16", 3, 48, 256, 113),
    "qmm_b4_g64_bf16_m40": lambda: case_qmm(4, 64, "bfloat16", 40, 96, 512, 114),
    "qmm_b4_g32_fp32_m2": lambda: case_qmm(4, 32, "float32", 2, 40, 160, 115),
    "rms_norm_bf16": lambda: case_rms("bfloat16", 5, 256, 1e-6, 121),
    "rms_norm_fp32": lambda: case_rms("float32", 3, 72, 1e-5, 122),
    "norm_rope_bf16": lambda: case_norm_rope("bfloat16", 6, 3, 64, 5, 131),
    "sdpa_causal_gqa_bf16": lambda: case_sdpa("bfloat16", 4, 2, 9, 64, 141),
    "swiglu_bf16": lambda: case_swiglu("bfloat16", 3, 70, 151),
    "shortconv_bf16": lambda: case_shortconv("bfloat16", 7, 48, False, 161),
    "shortconv_state_bf16": lambda: case_shortconv("bfloat16", 1, 48, True, 162),
    "tiny_mlp_fp32": lambda: case_tiny_mlp(4, 32, 64, 171),
    "argmax_bf16": lambda: case_argmax(1000, 181),
}


def build(name):
    meta, ins, outs = CASES[name]()
    arrays = {f"in_{k}": np.asarray(v) for k, v in ins.items()}
    arrays.update({f"out_{k}": np.asarray(v) for k, v in outs.items()})
    return meta, arrays


def load(name):
    """(meta, {name: array}) of a committed fixture."""
    with np.load(HERE / f"{name}.npz", allow_pickle=False) as z:
        arrays = {k: z[k] for k in z.files if k != "meta"}
        meta = json.loads(str(z["meta"]))
    return meta, arrays


def main():
    oracle.lib()
    for name in CASES:
        meta, arrays = build(name)
        np.savez_compressed(HERE / f"{name}.npz", meta=np.array(json.dumps(meta)), **arrays)
        print(f"{name}: {', '.join(f'{k}{list(v.shape)}' for k, v in arrays.items())}")


if __name__ == "__main__":
    main()
