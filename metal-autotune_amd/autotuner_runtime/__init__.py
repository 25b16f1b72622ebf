"""MI355X (gfx950) runtime for metal-autotune's quantized-matmul region path.

A torch/HIP mirror of the reference's ``autotuner_runtime`` package
(shivamg05/metal-autotune): the region API (``kernels``: KernelSpec,
load_spec, call / try_call / try_sized / fallback_fires; ``grammar``;
``stages``), the verifiers (``exact``, ``numeric``) and the install path
(``swap``, ``apply``), with the kernels behind them being hand-written HIP for
gfx950 (``hip`` binds the C ABI of include/mi_qmm.h; ``ops`` exposes the
library-level ops; ``regions`` holds the region specs of the reference's cuts).
"""

__all__ = ["apply", "exact", "grammar", "hip", "kernels", "numeric", "ops", "regions", "stages",
           "swap"]
