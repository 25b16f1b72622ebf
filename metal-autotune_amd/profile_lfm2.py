"""A fixed workload for kernel traces of config 5 (the LFM2 hybrid prefill).

    rocprofv3 --kernel-trace --stats --output-format csv -d OUT -o lfm2 -- python3 metal-autotune_amd/profile_lfm2.py

Builds the LFM2-1.2B-shaped model of bench.py's ``lfm2_config5`` (16 layers:
10 gated short-conv and 6 attention, hidden 2048, SwiGLU 8192, tied
V = 65536; ``--bits`` 4 or 8, random weights, seed 0) with the region cuts
installed. It captures one prefill of 2048 seeded token ids (greedy argmax on
the last position) as a HIP graph, replays it 3 times untimed, then times
``--reps`` replays with HIP events and prints the mean ms per prefill.
"""

from __future__ import annotations

import argparse
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT.parent))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--bits", type=int, default=4, choices=(4, 8))
    ap.add_argument("--reps", type=int, default=5)
    args = ap.parse_args()

    import torch

    import bench
    from autotuner_runtime import ops
    from workloads import lfm2, qwen3

    cfg = lfm2.Lfm2Config(bits=args.bits)
    model = lfm2.build(cfg, seed=0)
    lfm2.install_regions(model)
    ids = qwen3.tokens(2, 2048, cfg.vocab_size)
    caches = model.make_cache(2048)

    def step():
        for c in caches:
            c.offset = 0
            if isinstance(c, lfm2.ConvCache):
                c.state = None
        return ops.argmax(model(ids, caches).reshape(1, -1))

    g, _ = bench.graph_of(step, torch)
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    print(f"ms per prefill ({args.bits}-bit): {bench.time_graph(g, args.reps, torch):.3f}",
          flush=True)


if __name__ == "__main__":
    main()
