"""flash-mHC for MI355X: the mHC-lite K1/K3/K4 fused path on gfx950 HIP kernels.

Importing the package registers the ``torch.ops.flash_mhc.*`` custom ops.
The HIP extension itself is loaded on first use (see ``flash_mhc._abi``).
"""

from .block import MHCLiteBlock, build_permutation_matrices
from . import ops as _ops  # noqa: F401  # registers the torch.library ops

__all__ = ["MHCLiteBlock", "build_permutation_matrices"]
