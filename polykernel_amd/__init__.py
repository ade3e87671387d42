"""polykernel_amd -- MI355X (gfx950) fused transformer-block kernels.

The compute lives in libpolykernel_amd.so (hand-written HIP for gfx950 behind
the C-ABI of include/polykernel_amd.h).  `kernels` is the torch-tensor front
end, `runtime` the detect -> select -> serve layer with the tuning cache, and
`synth` / `metrics` the deterministic inputs and the correctness gate.
"""
from ._lib import LIB_PATH, PolyKernelError, load  # noqa: F401

__version__ = "0.1.0"
