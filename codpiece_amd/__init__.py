"""MI355X-native verify step for codpiece: HIP kernels behind a C ABI (libcpv.so).

The package is a thin host layer: `runtime.Context` wraps the C ABI of
include/cpv.h (the GEMM, attention, distribution and acceptance entry
points: codpiece-sample's interface among them); `model` mirrors
codpiece-model's verify-round interface and holds the greedy and sampled
speculative loops; `gguf` reads and writes the model files.  All arithmetic
runs in libcpv.so.
"""
from ._lib import (ACCEPT_GREEDY, ACCEPT_GUMBEL, ACCEPT_REJECT, F16, F32, Q4_K, Q6_K, Q8_0, CpvError,
                   SamplerParams, load)

__all__ = ["load", "CpvError", "SamplerParams", "F32", "F16", "Q8_0", "Q4_K", "Q6_K",
           "ACCEPT_GREEDY", "ACCEPT_REJECT", "ACCEPT_GUMBEL"]
