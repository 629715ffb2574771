"""drift_amd: the drift runner's fused layer kernels for MI355X (gfx950).

The kernels are hand-written HIP in `csrc/`, built into `libdrift_kernels.so`
beside this file and exported through the C ABI of include/drift_kernels.h.
`drift_amd.ops.HipOps` is the runner's `Ops` interface over them.
"""

from ._lib import HipError, NotBuilt, load  # noqa: F401

__all__ = ["HipError", "NotBuilt", "load"]
