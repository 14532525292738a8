"""Backward launchers over the gfx950 HIP kernels.

Same names and arguments as the reference's src/mhc/_backward.py:503-626.
Differences, both deliberate:

* weight gradients (dH_pre, dH_res, dH_post) keep the dtype of the weights they
  differentiate (fp32 in the module) instead of being rounded to H's dtype
  (reference :573,623-624) -- the autograd engine would cast them back to the
  weights' dtype anyway, so the rounding only lost precision;
* ``add_residual_backward`` returns ``dH_new`` itself as ``dH_residual`` (the
  identity gradient) instead of a copy (reference :333-337).
The reductions are deterministic two-level (wave shuffle + LDS, then a
fixed-order sum of per-workgroup partials) instead of partial buffers plus
``torch.sum``.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib
from ._kernels import ShapeError, _f32


def sinkhorn_backward(M_orig: torch.Tensor, dP: torch.Tensor, num_iters: int = 20,
                      eps: float = 1e-8) -> torch.Tensor:
    """Gradient of Sinkhorn-Knopp w.r.t. its input (reference
    src/mhc/_backward.py:503-530), in M_orig's dtype.  d|M|/dM uses sgn(0) = 0."""
    if tuple(M_orig.shape[-2:]) != (4, 4) or M_orig.shape != dP.shape:
        raise ShapeError(f"M_orig and dP must both be (..., 4, 4); got {tuple(M_orig.shape)}, {tuple(dP.shape)}")
    dev = _lib.require_gpu(M_orig, dP)
    M_orig = M_orig.contiguous()
    dP = dP.contiguous()
    dM = torch.empty_like(M_orig)
    lib = _lib.load()
    with _lib.on_device(dev):
        _lib.check(lib.mhc_sinkhorn_backward(M_orig.data_ptr(), _lib.dtype_code(M_orig), dP.data_ptr(),
                                             _lib.dtype_code(dP), dM.data_ptr(), M_orig.numel() // 16,
                                             int(num_iters), float(eps), _lib.stream(dev)), "sinkhorn_backward")
    return dM


def add_residual_backward(dH_new: torch.Tensor, branch_output: torch.Tensor, H_post: torch.Tensor,
                          block_dim: int = 128) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dH_residual, d_branch_output, dH_post) of H_new = H_residual + H_post*bo
    (reference src/mhc/_backward.py:533-575)."""
    B, S, _, D = dH_new.shape
    if tuple(branch_output.shape) != (B, S, D) or tuple(H_post.shape) != (B, 4):
        raise ShapeError("add_residual_backward: shape mismatch")
    dev = _lib.require_gpu(dH_new, branch_output, H_post)
    dH_new = dH_new.contiguous()
    branch_output = branch_output.contiguous()
    post = _f32(H_post)
    d_bo = torch.empty_like(branch_output)
    dH_post = torch.empty(B, 4, device=dev, dtype=torch.float32)
    lib = _lib.load()
    ws = _lib.workspace(lib.mhc_add_residual_backward_workspace_bytes(B, S, D, _lib.dtype_code(dH_new)), dev)
    with _lib.on_device(dev):
        _lib.check(lib.mhc_add_residual_backward(
            dH_new.data_ptr(), _lib.dtype_code(dH_new), branch_output.data_ptr(), _lib.dtype_code(branch_output),
            post.data_ptr(), d_bo.data_ptr(), dH_post.data_ptr(), B, S, D, _lib.ptr(ws),
            0 if ws is None else ws.numel(), _lib.stream(dev)), "add_residual_backward")
    return dH_new, d_bo, dH_post.to(H_post.dtype)


def stream_mix_backward(d_branch_input: torch.Tensor, dH_residual: torch.Tensor, H: torch.Tensor,
                        H_pre: torch.Tensor, H_res: torch.Tensor,
                        block_dim: int = 128) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dH, dH_pre, dH_res) of the stream mix (reference
    src/mhc/_backward.py:578-626)."""
    B, S, _, D = H.shape
    dev = _lib.require_gpu(d_branch_input, dH_residual, H, H_pre, H_res)
    dt = H.dtype
    d_branch_input = d_branch_input.contiguous().to(dt)
    dH_residual = dH_residual.contiguous().to(dt)
    H = H.contiguous()
    pre = _f32(H_pre)
    res = _f32(H_res)
    dH = torch.empty_like(H)
    dH_pre = torch.empty(B, 4, device=dev, dtype=torch.float32)
    dH_res = torch.empty(B, 4, 4, device=dev, dtype=torch.float32)
    lib = _lib.load()
    code = _lib.dtype_code(H)
    ws = _lib.workspace(lib.mhc_stream_mix_backward_workspace_bytes(B, S, D, code), dev)
    with _lib.on_device(dev):
        _lib.check(lib.mhc_stream_mix_backward(
            d_branch_input.data_ptr(), dH_residual.data_ptr(), H.data_ptr(), pre.data_ptr(), res.data_ptr(),
            dH.data_ptr(), dH_pre.data_ptr(), dH_res.data_ptr(), B, S, D, code, _lib.ptr(ws),
            0 if ws is None else ws.numel(), _lib.stream(dev)), "stream_mix_backward")
    return dH, dH_pre.to(H_pre.dtype), dH_res.to(H_res.dtype)


def fused_dynamic_weights_backward(x: torch.Tensor, phi: torch.Tensor, bias: torch.Tensor,
                                   alphas, aux: torch.Tensor, H_pre: torch.Tensor,
                                   grad_H_pre: Optional[torch.Tensor], grad_H_post: Optional[torch.Tensor],
                                   grad_H_res: Optional[torch.Tensor], sinkhorn_iters: int, eps: float):
    """All gradients of Eq. 14-19 (replaces the torch math of the reference's
    _FusedDynamicWeights.backward, src/mhc/ops.py:110-228).  grad_x comes back
    in x's dtype, as the reference casts it (ops.py:218-228); the parameter
    gradients are f32.  Returns (grad_x, grad_phi, grad_bias, grad_alpha[3])."""
    R, K = x.shape
    dev = _lib.require_gpu(x, phi, bias, aux, H_pre)
    x = x.contiguous()
    phi = _f32(phi)
    bias = _f32(bias)
    gx = torch.empty(R, K, device=dev, dtype=x.dtype)
    gphi = torch.empty(K, 24, device=dev, dtype=torch.float32)
    gbias = torch.empty(24, device=dev, dtype=torch.float32)
    galpha = torch.empty(3, device=dev, dtype=torch.float32)
    g = [None if t is None else _f32(t) for t in (grad_H_pre, grad_H_post, grad_H_res)]
    lib = _lib.load()
    ws = _lib.workspace(lib.mhc_dynamic_weights_backward_workspace_bytes(R, K), dev)
    with _lib.on_device(dev):
        _lib.check(lib.mhc_dynamic_weights_backward(
            x.data_ptr(), _lib.dtype_code(x), phi.data_ptr(), bias.data_ptr(),
            alphas[0].data_ptr(), alphas[1].data_ptr(), alphas[2].data_ptr(), aux.data_ptr(), H_pre.data_ptr(),
            _lib.ptr(g[0]), _lib.ptr(g[1]), _lib.ptr(g[2]), gx.data_ptr(), gphi.data_ptr(), gbias.data_ptr(),
            galpha.data_ptr(), R, K, int(sinkhorn_iters), float(eps), _lib.ptr(ws),
            0 if ws is None else ws.numel(), _lib.stream(dev)), "dynamic_weights_backward")
    return gx, gphi, gbias, galpha
