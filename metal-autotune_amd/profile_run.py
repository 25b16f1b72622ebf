"""A fixed kernel workload for hardware-counter passes (rocprofv3 --pmc).

    rocprofv3 --pmc FETCH_SIZE -d OUT -o dual -- python metal-autotune_amd/profile_run.py
    rocprofv3 --pmc WRITE_SIZE -d OUT -o dual -- python metal-autotune_amd/profile_run.py

Runs, eagerly on the current stream:

1. ``copies`` launches of a plain device copy of COPY_BYTES (torch's
   elementwise copy kernel): the calibration that says how many KiB the
   FETCH_SIZE / WRITE_SIZE counters report per byte actually moved;
2. ``reps`` launches of the prefill gate/up region kernel (dual 4-bit qmm with
   the SwiGLU epilogue, x[128, 2560] against two [9728, 2560] weights, group
   64) rotating over enough weight sets that they cannot stay in the 256 MB
   Infinity Cache -- the same kernel and shape bench.py reports in
   ``roofline``;
3. the same for a plain qmm at M = 1 (decode GEMV, [9728, 2560]);
4. the two narrow projections of the layer with their residual epilogue
   (``ops.qmm_residual``, the [qmm, add] region): o_proj (x[128, 4096] @
   [2560, 4096]^T) and down_proj (x[128, 9728] @ [2560, 9728]^T), each over
   enough weight copies to exceed the Infinity Cache;
5. the fused q/k/v + q/k-norm + RoPE + cache write (``ops.qkv_norm_rope``,
   32 q / 8 kv heads of 128 from x[128, 2560]) likewise;
6. the LFM2 prefill's gate/up region: dual 4-bit qmm + SwiGLU at M = 2048
   (x[2048, 2048] against two [8192, 2048] weights, group 64; the interleaved
   K split), over enough weight sets to exceed the Infinity Cache.

Prints one line per phase so the counter rows can be matched to phases by
kernel name and launch order.
"""

from __future__ import annotations

import argparse
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parent))

COPY_BYTES = 256 << 20


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reps", type=int, default=24)
    ap.add_argument("--copies", type=int, default=4)
    args = ap.parse_args()

    import torch

    from autotuner_runtime import hip, ops
    from workloads.quantize import random_quantized

    hip.lib()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(11)
    src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device="cuda").uniform_(generator=gen)
    dst = torch.empty_like(src)
    for _ in range(args.copies):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"phase copy: {args.copies} x {COPY_BYTES} bytes read + written", flush=True)
    del src, dst

    N, K, M = 9728, 2560, 128
    sets = 12  # 12 x 2 x 13.2 MB > 256 MB
    ws = [(random_quantized(N, K, gen, "cuda"), random_quantized(N, K, gen, "cuda"))
          for _ in range(sets)]
    x = torch.randn((1, M, K), generator=gen, device="cuda").to(torch.bfloat16)
    for i in range(args.reps):
        g, u = ws[i % sets]
        ops.qmm_dual(x, *g, *u, swiglu=True)
    torch.cuda.synchronize()
    print(f"phase dual: {args.reps} x qmm_dual swiglu M={M} N=2x{N} K={K}", flush=True)

    x1 = x[:, :1].contiguous()
    for i in range(args.reps):
        ops.quantized_matmul(x1, *ws[i % sets][i % 2])
    torch.cuda.synchronize()
    print(f"phase gemv: {args.reps} x qmm M=1 N={N} K={K}", flush=True)
    del ws

    for name, n_out, k_in in (("o_proj", 2560, 4096), ("down_proj", 2560, 9728)):
        per = n_out * k_in * 9 // 16
        copies = (300 << 20) // per + 1
        wsn = [random_quantized(n_out, k_in, gen, "cuda") for _ in range(copies)]
        xin = torch.randn((1, M, k_in), generator=gen, device="cuda").to(torch.bfloat16)
        res = torch.randn((1, M, n_out), generator=gen, device="cuda").to(torch.bfloat16)
        for i in range(args.reps):
            ops.qmm_residual(xin, *wsn[i % copies], res)
        torch.cuda.synchronize()
        print(f"phase {name}: {args.reps} x qmm+residual M={M} N={n_out} K={k_in}", flush=True)
        del wsn

    # the q/k/v projections with q/k-norm, RoPE and the cache write in one
    # launch (32 q / 8 kv heads of 128, K 2560), over enough weight copies
    H, HK, D = 32, 8, 128
    per = (H + 2 * HK) * D * K * 9 // 16
    copies = (300 << 20) // per + 1
    wq = [[random_quantized(n, K, gen, "cuda") for n in (H * D, HK * D, HK * D)]
          for _ in range(copies)]
    qn = torch.ones(D, dtype=torch.bfloat16, device="cuda")
    kc = torch.zeros((1, HK, M, D), dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    for i in range(args.reps):
        ops.qkv_norm_rope(x, wq[i % copies], qn, qn, H, HK, 1e-6, D, 1e6, 0, kc, vc, 0)
    torch.cuda.synchronize()
    print(f"phase qkv_norm_rope: {args.reps} x q/k/v + norm + rope M={M} heads {H}+{HK}+{HK} "
          f"D={D} K={K}", flush=True)
    del wq

    N, K, M = 8192, 2048, 2048
    sets = 16  # 16 x 2 x 9.4 MB > 256 MB
    ws = [(random_quantized(N, K, gen, "cuda"), random_quantized(N, K, gen, "cuda"))
          for _ in range(sets)]
    x = torch.randn((1, M, K), generator=gen, device="cuda").to(torch.bfloat16)
    for i in range(args.reps):
        g, u = ws[i % sets]
        ops.qmm_dual(x, *g, *u, swiglu=True)
    torch.cuda.synchronize()
    print(f"phase dual2048: {args.reps} x qmm_dual swiglu M={M} N=2x{N} K={K}", flush=True)


if __name__ == "__main__":
    main()
