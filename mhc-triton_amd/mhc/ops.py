"""High-level ops with autograd support (reference src/mhc/ops.py).

Same Function names, forward signatures, outputs and gradient signatures as the
reference; every forward and backward runs on the gfx950 HIP kernels.
"""

from __future__ import annotations

from typing import Tuple

import torch

from . import _backward as _bwd
from . import _kernels as _k
from . import _library  # noqa: F401  (registers torch.ops.mhc.*)


class _SinkhornKnopp(torch.autograd.Function):
    """Sinkhorn-Knopp projection (reference src/mhc/ops.py:15-29)."""

    @staticmethod
    def forward(ctx, M: torch.Tensor, num_iters: int, eps: float) -> torch.Tensor:
        ctx.save_for_backward(M)
        ctx.num_iters = num_iters
        ctx.eps = eps
        return _k.sinkhorn_forward(M, num_iters, eps)

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        M, = ctx.saved_tensors
        return _bwd.sinkhorn_backward(M, grad_output, ctx.num_iters, ctx.eps), None, None


class _FusedStreamMix(torch.autograd.Function):
    """Stream mix, Eq. 10-11 (reference src/mhc/ops.py:32-49)."""

    @staticmethod
    def forward(ctx, H: torch.Tensor, H_pre: torch.Tensor, H_res: torch.Tensor):
        branch_input, H_residual = _k.stream_mix_forward(H, H_pre, H_res)
        ctx.save_for_backward(H, H_pre, H_res)
        return branch_input, H_residual

    @staticmethod
    def backward(ctx, grad_branch_input: torch.Tensor, grad_H_residual: torch.Tensor):
        H, H_pre, H_res = ctx.saved_tensors
        return _bwd.stream_mix_backward(grad_branch_input, grad_H_residual, H, H_pre, H_res)


class _FusedAddResidual(torch.autograd.Function):
    """Add residual, Eq. 12 (reference src/mhc/ops.py:52-69)."""

    @staticmethod
    def forward(ctx, H_residual: torch.Tensor, branch_output: torch.Tensor, H_post: torch.Tensor):
        H_new = _k.add_residual_forward(H_residual, branch_output, H_post)
        ctx.save_for_backward(branch_output, H_post)
        return H_new

    @staticmethod
    def backward(ctx, grad_H_new: torch.Tensor):
        branch_output, H_post = ctx.saved_tensors
        return _bwd.add_residual_backward(grad_H_new, branch_output, H_post)


class _FusedDynamicWeights(torch.autograd.Function):
    """Dynamic weights, Eq. 14-19 (reference src/mhc/ops.py:72-228).

    Forward and backward are both HIP kernels; the alphas stay on the device
    (the reference calls ``.item()`` on each, ops.py:98).
    """

    @staticmethod
    def forward(ctx, x, phi, bias, alpha_pre, alpha_post, alpha_res, sinkhorn_iters: int, eps: float):
        H_pre, H_post, H_res, aux = _k.fused_dynamic_weights_forward(
            x, phi, bias, alpha_pre, alpha_post, alpha_res, sinkhorn_iters, eps, return_aux=True)
        ctx.save_for_backward(x, phi, bias, alpha_pre, alpha_post, alpha_res, H_pre, aux)
        ctx.sinkhorn_iters = sinkhorn_iters
        ctx.eps = eps
        ctx.set_materialize_grads(False)
        return H_pre, H_post, H_res

    @staticmethod
    def backward(ctx, grad_H_pre, grad_H_post, grad_H_res):
        x, phi, bias, a_pre, a_post, a_res, H_pre, aux = ctx.saved_tensors
        alphas = [_k._alpha_tensor(a, x.device) for a in (a_pre, a_post, a_res)]
        gx, gphi, gbias, galpha = _bwd.fused_dynamic_weights_backward(
            x, phi, bias, alphas, aux, H_pre, grad_H_pre, grad_H_post,
            None if grad_H_res is None else grad_H_res.reshape(-1, 16),
            ctx.sinkhorn_iters, ctx.eps)
        return (
            gx.to(x.dtype),
            gphi.to(phi.dtype),
            gbias.to(bias.dtype),
            galpha[0:1].reshape(a_pre.shape).to(a_pre.dtype),
            galpha[1:2].reshape(a_post.shape).to(a_post.dtype),
            galpha[2:3].reshape(a_res.shape).to(a_res.dtype),
            None,
            None,
        )


def sinkhorn_knopp(M: torch.Tensor, num_iters: int = 20, eps: float = 1e-8) -> torch.Tensor:
    """Project (batch, 4, 4) matrices to doubly stochastic via Sinkhorn-Knopp."""
    if torch.compiler.is_compiling():
        return torch.ops.mhc.sinkhorn_forward(M, num_iters, eps)
    return _SinkhornKnopp.apply(M, num_iters, eps)


def fused_stream_mix(H: torch.Tensor, H_pre: torch.Tensor, H_res: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """branch_input (batch, seq, dim) and H_residual (batch, seq, 4, dim) of H (batch, seq, 4, dim)."""
    if torch.compiler.is_compiling():
        return torch.ops.mhc.stream_mix_forward(H, H_pre, H_res)
    return _FusedStreamMix.apply(H, H_pre, H_res)


def fused_add_residual(H_residual: torch.Tensor, branch_output: torch.Tensor, H_post: torch.Tensor) -> torch.Tensor:
    """H_new[n] = H_residual[n] + H_post[n] * branch_output."""
    if torch.compiler.is_compiling():
        return torch.ops.mhc.add_residual_forward(H_residual, branch_output, H_post)
    return _FusedAddResidual.apply(H_residual, branch_output, H_post)


def fused_dynamic_weights(
    x: torch.Tensor,
    phi: torch.Tensor,
    bias: torch.Tensor,
    alpha_pre: torch.Tensor,
    alpha_post: torch.Tensor,
    alpha_res: torch.Tensor,
    sinkhorn_iters: int = 20,
    eps: float = 1e-6,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(H_pre [batch,4], H_post [batch,4], H_res [batch,4,4]) from x [batch, 4*dim] (Eq. 14-19)."""
    if torch.compiler.is_compiling():
        alphas = [a if isinstance(a, torch.Tensor) else torch.tensor([float(a)], device=x.device)
                  for a in (alpha_pre, alpha_post, alpha_res)]
        return torch.ops.mhc.dynamic_weights_forward(x, phi, bias, *alphas, sinkhorn_iters, eps)[:3]
    return _FusedDynamicWeights.apply(x, phi, bias, alpha_pre, alpha_post, alpha_res, sinkhorn_iters, eps)
