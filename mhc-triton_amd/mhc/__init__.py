"""mhc -- Manifold-Constrained Hyper-Connections on MI355X (gfx950 HIP kernels).

Drop-in for the ``mhc`` package of WithNucleusAI/mHC-triton (reference
src/mhc/__init__.py): the same names, signatures and autograd behaviour, with
every op running on hand-written HIP kernels behind the C ABI of
``libmhc_hip.so`` (include/mhc_abi.h).  The ``*_torch`` baselines are plain
PyTorch and run anywhere.
"""

from . import streams  # stream expand / collapse (not in __all__, which is the reference's)
from .module import HyperConnection
from .ops import (
    sinkhorn_knopp,
    fused_stream_mix,
    fused_add_residual,
    fused_dynamic_weights,
)
from ._torch_baseline import (
    sinkhorn_knopp_torch,
    fused_stream_mix_torch,
    fused_add_residual_torch,
    fused_dynamic_weights_torch,
    HyperConnectionTorch,
)

__version__ = "0.1.0"
__all__ = [
    "HyperConnection",
    "sinkhorn_knopp",
    "fused_stream_mix",
    "fused_add_residual",
    "fused_dynamic_weights",
    # PyTorch baselines for benchmarking
    "sinkhorn_knopp_torch",
    "fused_stream_mix_torch",
    "fused_add_residual_torch",
    "fused_dynamic_weights_torch",
    "HyperConnectionTorch",
]
