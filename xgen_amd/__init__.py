"""xgen_amd — MI355X (gfx950) native quantized DiT linear path.

Host side in Python on PyTorch-ROCm; compute in hand-written HIP kernels
(xgen_amd/csrc) behind a C ABI (include/xgen_amd.h), exposed as torch.library
operators (xgen_amd.ops) and as modules with the reference's surface
(xgen_amd.operator.*).  Importing the package registers the operators; the
HIP library is loaded on first use.
"""
from . import ops  # noqa: F401  (registers torch.ops.xgen_amd.*)
from . import reference_ops  # noqa: F401  (registers the reference's torch.ops.h3_phaa_* fused ops)
from ._native import library_path  # noqa: F401

__all__ = ["ops", "reference_ops", "library_path"]
