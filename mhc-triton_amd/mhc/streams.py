"""Stream expand / collapse: the two ends of a hyper-connection stack.

The reference's ``HyperConnection`` takes the hyper-hidden state H
(batch, seq, 4, dim) as given (README.md:38-39) and leaves it to the caller to
build H from the embeddings and to reduce it at the model output.  These two
ops do that on the HIP kernels (``mhc_stream_expand`` / ``mhc_stream_collapse``):

    H = expand_streams(embeddings)          # (B, S, D) -> (B, S, 4, D)
    for block in blocks: H = block(H)       # HyperConnection layers
    h = collapse_streams(H)                 # (B, S, 4, D) -> (B, S, D), stream mean

Each is the other's backward (they are adjoint), so gradients cost one more
pass of the same kernel.  Not part of ``mhc.__all__``, which stays the
reference's.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _kernels as _k
from . import _library  # noqa: F401  (registers torch.ops.mhc.*)

__all__ = ["expand_streams", "collapse_streams"]

_REDUCTIONS = {"sum": 1.0, "mean": 0.25}


class _StreamExpand(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, scale: float, dtype):
        ctx.scale = scale
        ctx.x_dtype = x.dtype
        return _k.stream_expand(x, scale, dtype)

    @staticmethod
    def backward(ctx, dH):
        return _k.stream_collapse(dH, ctx.scale, ctx.x_dtype), None, None


class _StreamCollapse(torch.autograd.Function):
    @staticmethod
    def forward(ctx, H, scale: float, dtype):
        ctx.scale = scale
        ctx.h_dtype = H.dtype
        return _k.stream_collapse(H, scale, dtype)

    @staticmethod
    def backward(ctx, dy):
        return _k.stream_expand(dy, ctx.scale, ctx.h_dtype), None, None


def expand_streams(x: torch.Tensor, num_streams: int = 4, scale: float = 1.0,
                   dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """(batch, seq, dim) -> (batch, seq, 4, dim): every stream starts as ``scale * x``."""
    if num_streams != 4:
        raise ValueError("HIP kernels require num_streams=4")
    if torch.compiler.is_compiling():
        return torch.ops.mhc.stream_expand(x, float(scale), dtype)
    return _StreamExpand.apply(x, float(scale), dtype)


def collapse_streams(H: torch.Tensor, reduction: str = "mean",
                     dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """(batch, seq, 4, dim) -> (batch, seq, dim): the stream mean (or sum)."""
    if reduction not in _REDUCTIONS:
        raise ValueError(f"reduction must be 'mean' or 'sum', got {reduction!r}")
    scale = _REDUCTIONS[reduction]
    if torch.compiler.is_compiling():
        return torch.ops.mhc.stream_collapse(H, scale, dtype)
    return _StreamCollapse.apply(H, scale, dtype)
