"""The vendor bf16 GEMM (torch.matmul -> hipBLASLt) at the Qwen3 prefill
projection shapes (M = 128), as a yardstick for the 4-bit qmm kernels.

    python metal-autotune_amd/profile_hipblaslt.py

Weights are bf16 (3.6x the bytes of the 4-bit ones), rotated over more copies
than the 256 MB Infinity Cache holds; x is [128, K] bf16. Prints one line per
shape: HIP-event time per call (20 calls per copy, back to back), TFLOP/s and
the fraction of the 2.5 PFLOP/s dense bf16 peak.
"""

import torch, time
torch.manual_seed(0)
dev = "cuda"
M = 128
shapes = [("dual(gate+up)", 19456, 2560), ("gate", 9728, 2560), ("qkv", 6144, 2560),
          ("o_proj", 2560, 4096), ("down", 2560, 9728)]
for name, N, K in shapes:
    per = N * K * 2
    copies = max(2, (1 << 30) // per + 1)
    ws = [torch.randn(N, K, device=dev, dtype=torch.bfloat16) for _ in range(copies)]
    x = torch.randn(M, K, device=dev, dtype=torch.bfloat16)
    for i in range(10):
        y = x @ ws[i % copies].t()
    torch.cuda.synchronize()
    n = 20 * copies
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(n):
        y = x @ ws[i % copies].t()
    e1.record(); e1.synchronize()
    us = e0.elapsed_time(e1) * 1000 / n
    fl = 2 * M * N * K
    print(f"{name:14s} M={M} N={N} K={K}: {us:7.2f} us  {fl/us/1e6:7.1f} TFLOP/s  {100*fl/us/1e6/2500:5.1f}% of bf16 peak  "
          f"(bf16 weights {per/us/1e3:6.0f} GB/s)", flush=True)
    del ws
