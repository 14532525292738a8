"""torch.library registrations of the HIP entry points (namespace ``mhc``).

torch.compile cannot trace through the ctypes calls of the eager launchers, so
each launcher is also registered as a custom op with a fake implementation
(output shapes and dtypes only).  Traced code then sees opaque ``torch.ops.mhc.*``
nodes and compiles the whole graph around them without a graph break.

* The four public ops (reference src/mhc/ops.py:231-323) and the mean-pool
  carry their backward as ``torch.library.register_autograd`` formulas that call
  the backward ops.
* The layer (reference src/mhc/module.py:103-182) uses the same two autograd
  nodes as eager mode (``_layer.py``), on the custom ops: node A returns a view
  of ``H`` (the *link*) and an unwritten [B,4] tensor (the *post link*) that only
  the closure consumes; the closure's backward returns ``dH_new`` and ``dH_post``
  as their gradients, and node A writes the complete ``dH`` in one pass.

Eager calls keep going through the launchers directly: a custom-op dispatch
costs about 13 us of host time, more than some of the kernels it would wrap.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from . import _backward as _b
from . import _kernels as _k
from . import _layer as _l

_F32 = torch.float32


def _op(name: str):
    return torch.library.custom_op(f"mhc::{name}", mutates_args=(), device_types="cuda")


def _f32_like(ref: Tensor, *shape) -> Tensor:
    return ref.new_empty(shape, dtype=_F32)


# --------------------------------------------------------------------------
# Sinkhorn-Knopp (reference _kernels.py:597, _backward.py:503)
# --------------------------------------------------------------------------

@_op("sinkhorn_forward")
def sinkhorn_forward(M: Tensor, num_iters: int, eps: float) -> Tensor:
    return _k.sinkhorn_forward(M, num_iters, eps)


@sinkhorn_forward.register_fake
def _(M, num_iters, eps):
    return M.new_empty(M.shape)


@_op("sinkhorn_backward")
def sinkhorn_backward(M: Tensor, dP: Tensor, num_iters: int, eps: float) -> Tensor:
    return _b.sinkhorn_backward(M, dP, num_iters, eps)


@sinkhorn_backward.register_fake
def _(M, dP, num_iters, eps):
    return M.new_empty(M.shape)


def _sinkhorn_setup(ctx, inputs, output):
    M, num_iters, eps = inputs
    ctx.save_for_backward(M)
    ctx.num_iters = num_iters
    ctx.eps = eps


def _sinkhorn_bwd(ctx, dP):
    M, = ctx.saved_tensors
    return torch.ops.mhc.sinkhorn_backward(M, dP, ctx.num_iters, ctx.eps), None, None


torch.library.register_autograd("mhc::sinkhorn_forward", _sinkhorn_bwd, setup_context=_sinkhorn_setup)


# --------------------------------------------------------------------------
# Stream mix (reference _kernels.py:617, _backward.py:578)
# --------------------------------------------------------------------------

@_op("stream_mix_forward")
def stream_mix_forward(H: Tensor, H_pre: Tensor, H_res: Tensor) -> Tuple[Tensor, Tensor]:
    return _k.stream_mix_forward(H, H_pre, H_res)


@stream_mix_forward.register_fake
def _(H, H_pre, H_res):
    B, S, _, D = H.shape
    return H.new_empty(B, S, D), H.new_empty(H.shape)


@_op("stream_mix_backward")
def stream_mix_backward(d_branch_input: Tensor, dH_residual: Tensor, H: Tensor, H_pre: Tensor,
                        H_res: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
    return _b.stream_mix_backward(d_branch_input, dH_residual, H, H_pre, H_res)


@stream_mix_backward.register_fake
def _(d_branch_input, dH_residual, H, H_pre, H_res):
    B = H.shape[0]
    return H.new_empty(H.shape), H_pre.new_empty(B, 4), H_res.new_empty(B, 4, 4)


def _mix_setup(ctx, inputs, output):
    ctx.save_for_backward(*inputs)


def _mix_bwd(ctx, d_bi, d_res):
    H, H_pre, H_res = ctx.saved_tensors
    if d_bi is None:
        d_bi = H.new_zeros(H.shape[0], H.shape[1], H.shape[3])
    if d_res is None:
        d_res = torch.zeros_like(H)
    return torch.ops.mhc.stream_mix_backward(d_bi, d_res, H, H_pre, H_res)


torch.library.register_autograd("mhc::stream_mix_forward", _mix_bwd, setup_context=_mix_setup)


# --------------------------------------------------------------------------
# Add residual (reference _kernels.py:655, _backward.py:533)
# --------------------------------------------------------------------------

@_op("add_residual_forward")
def add_residual_forward(H_residual: Tensor, branch_output: Tensor, H_post: Tensor) -> Tensor:
    return _k.add_residual_forward(H_residual, branch_output, H_post)


@add_residual_forward.register_fake
def _(H_residual, branch_output, H_post):
    return H_residual.new_empty(H_residual.shape)


@_op("add_residual_backward")
def add_residual_backward(dH_new: Tensor, branch_output: Tensor, H_post: Tensor) -> Tuple[Tensor, Tensor]:
    """(d_branch_output, dH_post); dH_residual is dH_new itself and is not an output."""
    _, d_bo, dpost = _b.add_residual_backward(dH_new, branch_output, H_post)
    return d_bo, dpost


@add_residual_backward.register_fake
def _(dH_new, branch_output, H_post):
    return branch_output.new_empty(branch_output.shape), H_post.new_empty(dH_new.shape[0], 4)


def _add_setup(ctx, inputs, output):
    H_residual, bo, H_post = inputs
    ctx.save_for_backward(bo, H_post)


def _add_bwd(ctx, dH_new):
    bo, H_post = ctx.saved_tensors
    d_bo, dpost = torch.ops.mhc.add_residual_backward(dH_new, bo, H_post)
    return dH_new, d_bo, dpost


torch.library.register_autograd("mhc::add_residual_forward", _add_bwd, setup_context=_add_setup)


# --------------------------------------------------------------------------
# Dynamic weights (reference _kernels.py:690, ops.py:72-228)
# --------------------------------------------------------------------------

@_op("dynamic_weights_forward")
def dynamic_weights_forward(x: Tensor, phi: Tensor, bias: Tensor, alpha_pre: Tensor, alpha_post: Tensor,
                            alpha_res: Tensor, sinkhorn_iters: int,
                            eps: float) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """(H_pre [R,4], H_post [R,4], H_res [R,4,4], aux [R,25]), all f32."""
    return _k.fused_dynamic_weights_forward(x, phi, bias, alpha_pre, alpha_post, alpha_res, sinkhorn_iters,
                                            eps, return_aux=True)


@dynamic_weights_forward.register_fake
def _(x, phi, bias, alpha_pre, alpha_post, alpha_res, sinkhorn_iters, eps):
    R = x.shape[0]
    return _f32_like(x, R, 4), _f32_like(x, R, 4), _f32_like(x, R, 4, 4), _f32_like(x, R, 25)


@_op("dynamic_weights_backward")
def dynamic_weights_backward(x: Tensor, phi: Tensor, bias: Tensor, alpha_pre: Tensor, alpha_post: Tensor,
                             alpha_res: Tensor, aux: Tensor, H_pre: Tensor, grad_H_pre: Optional[Tensor],
                             grad_H_post: Optional[Tensor], grad_H_res: Optional[Tensor], sinkhorn_iters: int,
                             eps: float) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """(grad_x in x's dtype, grad_phi [K,24], grad_bias [24], grad_alpha [3]), parameter grads f32."""
    alphas = [_k._alpha_tensor(a, x.device) for a in (alpha_pre, alpha_post, alpha_res)]
    return _b.fused_dynamic_weights_backward(
        x, phi, bias, alphas, aux, H_pre, grad_H_pre, grad_H_post,
        None if grad_H_res is None else grad_H_res.reshape(-1, 16), sinkhorn_iters, eps)


@dynamic_weights_backward.register_fake
def _(x, phi, bias, alpha_pre, alpha_post, alpha_res, aux, H_pre, grad_H_pre, grad_H_post, grad_H_res,
      sinkhorn_iters, eps):
    R, K = x.shape
    return x.new_empty(R, K), _f32_like(x, K, 24), _f32_like(x, 24), _f32_like(x, 3)


def _dynw_setup(ctx, inputs, output):
    x, phi, bias, a_pre, a_post, a_res, iters, eps = inputs
    H_pre, _, _, aux = output
    ctx.save_for_backward(x, phi, bias, a_pre, a_post, a_res, H_pre, aux)
    ctx.iters = iters
    ctx.eps = eps
    ctx.mark_non_differentiable(aux)
    ctx.set_materialize_grads(False)


def _dynw_bwd(ctx, g_pre, g_post, g_res, g_aux):
    x, phi, bias, a_pre, a_post, a_res, H_pre, aux = ctx.saved_tensors
    gx, gphi, gbias, galpha = torch.ops.mhc.dynamic_weights_backward(
        x, phi, bias, a_pre, a_post, a_res, aux, H_pre, g_pre, g_post, g_res, ctx.iters, ctx.eps)
    return (gx, gphi.to(phi.dtype), gbias.to(bias.dtype),
            galpha[0:1].reshape(a_pre.shape).to(a_pre.dtype), galpha[1:2].reshape(a_post.shape).to(a_post.dtype),
            galpha[2:3].reshape(a_res.shape).to(a_res.dtype), None, None)


torch.library.register_autograd("mhc::dynamic_weights_forward", _dynw_bwd, setup_context=_dynw_setup)


# --------------------------------------------------------------------------
# Mean-pool (reference module.py:123)
# --------------------------------------------------------------------------

@_op("mean_pool")
def mean_pool(H: Tensor) -> Tensor:
    """x [B, 4*dim] f32 = mean of H over the sequence, stream-major."""
    return _k.mean_pool(H)


@mean_pool.register_fake
def _(H):
    B, _, n, D = H.shape
    return _f32_like(H, B, n * D)


def _pool_setup(ctx, inputs, output):
    H, = inputs
    ctx.shape = H.shape
    ctx.dtype = H.dtype


def _pool_bwd(ctx, gx):
    B, S, n, D = ctx.shape
    return (gx / S).to(ctx.dtype).reshape(B, 1, n, D).expand(B, S, n, D)


torch.library.register_autograd("mhc::mean_pool", _pool_bwd, setup_context=_pool_setup)


# --------------------------------------------------------------------------
# Layer-level entry points (include/mhc_abi.h mhc_layer_*)
# --------------------------------------------------------------------------

@_op("layer_dynamic_forward")
def layer_dynamic_forward(H: Tensor, phi: Tensor, H_pre_base: Tensor, H_post_base: Tensor, H_res_base: Tensor,
                          alpha_pre: Tensor, alpha_post: Tensor, alpha_res: Tensor, iters: int,
                          eps: float) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """(branch_input, x [B,4D] f32, w [B,24] f32, aux [B,25] f32)."""
    return _l.dynamic_forward(H, phi, H_pre_base, H_post_base, H_res_base, alpha_pre, alpha_post, alpha_res,
                              iters, eps)


@layer_dynamic_forward.register_fake
def _(H, phi, H_pre_base, H_post_base, H_res_base, alpha_pre, alpha_post, alpha_res, iters, eps):
    B, S, _, D = H.shape
    return H.new_empty(B, S, D), _f32_like(H, B, 4 * D), _f32_like(H, B, 24), _f32_like(H, B, 25)


@_op("layer_dynamic_backward")
def layer_dynamic_backward(H: Tensor, d_bi: Optional[Tensor], dH_new: Optional[Tensor], dH_post: Optional[Tensor],
                           phi: Tensor, H_pre_base: Tensor, H_post_base: Tensor, H_res_base: Tensor,
                           alpha_pre: Tensor, alpha_post: Tensor, alpha_res: Tensor, x: Tensor, w: Tensor,
                           aux: Tensor, iters: int, eps: float) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """(dH, grad_phi [4D,24], grad_bias [24], grad_alpha [3]), parameter grads f32."""
    return _l.dynamic_backward(H, d_bi, dH_new, dH_post, phi, H_pre_base, H_post_base, H_res_base, alpha_pre,
                               alpha_post, alpha_res, x, w, aux, iters, eps)


@layer_dynamic_backward.register_fake
def _(H, d_bi, dH_new, dH_post, phi, H_pre_base, H_post_base, H_res_base, alpha_pre, alpha_post, alpha_res,
      x, w, aux, iters, eps):
    D = H.shape[3]
    return H.new_empty(H.shape), _f32_like(H, 4 * D, 24), _f32_like(H, 24), _f32_like(H, 3)


@_op("layer_static_forward")
def layer_static_forward(H: Tensor, H_pre_base: Tensor, H_post_base: Tensor, H_res_base: Tensor,
                         iters: int) -> Tuple[Tensor, Tensor]:
    """(branch_input, w [B,24] f32)."""
    return _l.static_forward(H, H_pre_base, H_post_base, H_res_base, iters)


@layer_static_forward.register_fake
def _(H, H_pre_base, H_post_base, H_res_base, iters):
    B, S, _, D = H.shape
    return H.new_empty(B, S, D), _f32_like(H, B, 24)


@_op("layer_static_backward")
def layer_static_backward(H: Tensor, d_bi: Optional[Tensor], dH_new: Optional[Tensor], dH_post: Optional[Tensor],
                          H_pre_base: Tensor, H_post_base: Tensor, H_res_base: Tensor, w: Tensor,
                          iters: int) -> Tuple[Tensor, Tensor]:
    """(dH, grad_bias [24] f32)."""
    return _l.static_backward(H, d_bi, dH_new, dH_post, H_pre_base, H_post_base, H_res_base, w, iters)


@layer_static_backward.register_fake
def _(H, d_bi, dH_new, dH_post, H_pre_base, H_post_base, H_res_base, w, iters):
    return H.new_empty(H.shape), _f32_like(H, 24)


@_op("layer_branch_input")
def layer_branch_input(H: Tensor, w: Tensor) -> Tensor:
    return _l.branch_input(H, w)


@layer_branch_input.register_fake
def _(H, w):
    B, S, _, D = H.shape
    return H.new_empty(B, S, D)


@_op("layer_mix_backward")
def layer_mix_backward(H: Tensor, d_bi: Optional[Tensor], dH_new: Optional[Tensor],
                       w: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
    """(dH, dH_pre [B,4] f32, dH_res [B,16] f32)."""
    return _l.mix_backward(H, d_bi, dH_new, w)


@layer_mix_backward.register_fake
def _(H, d_bi, dH_new, w):
    B = H.shape[0]
    return H.new_empty(H.shape), _f32_like(H, B, 4), _f32_like(H, B, 16)


@_op("layer_mix_reduce")
def layer_mix_reduce(H: Tensor, d_bi: Optional[Tensor], dH_new: Optional[Tensor], w: Tensor) -> Tuple[Tensor, Tensor]:
    """(dH_pre [B,4] f32, dH_res [B,16] f32): the reductions of layer_mix_backward without dH, on
    the same reduction-only pass as the eager layer."""
    _, dpre, dres = _l.mix_backward(H, d_bi, dH_new, w, need_dH=False)
    return dpre, dres


@layer_mix_reduce.register_fake
def _(H, d_bi, dH_new, w):
    B = H.shape[0]
    return _f32_like(H, B, 4), _f32_like(H, B, 16)


@_op("layer_mix_dh")
def layer_mix_dh(d_bi: Optional[Tensor], dH_new: Optional[Tensor], w: Tensor, grad_x: Optional[Tensor],
                 H: Tensor) -> Tensor:
    """dH = H_pre d_bi + H_res^T dH_new + grad_x / S in H's dtype (H gives shape and dtype only)."""
    return _l.mix_dh(d_bi, dH_new, w, grad_x, H.shape, H.dtype)


@layer_mix_dh.register_fake
def _(d_bi, dH_new, w, grad_x, H):
    return H.new_empty(H.shape)


@_op("layer_add_forward")
def layer_add_forward(H: Tensor, branch_output: Tensor, w: Tensor) -> Tensor:
    return _l.add_forward(H, branch_output, w)


@layer_add_forward.register_fake
def _(H, branch_output, w):
    return H.new_empty(H.shape)


@_op("layer_add_backward")
def layer_add_backward(dH_new: Tensor, branch_output: Tensor, w: Tensor) -> Tuple[Tensor, Tensor]:
    """(d_branch_output, dH_post [B,4] f32)."""
    return _l.add_backward(dH_new, branch_output, w)


@layer_add_backward.register_fake
def _(dH_new, branch_output, w):
    return branch_output.new_empty(branch_output.shape), _f32_like(dH_new, dH_new.shape[0], 4)


def snapshot_links(H: Tensor, w: Tensor):
    """The closure's gradient carriers in traced code: a snapshot of H (-> dH_new) and an
    unwritten [B, 4] tensor (-> dH_post).

    Eager mode passes a view of H and raises if H's version counter moved before the closure
    runs.  Traced code cannot guard on a version counter (dynamo makes it a data-dependent
    value), and under functionalization a view would see an in-place change of H made between
    forward and the closure call.  The snapshot keeps the reference's semantics, where the
    closure holds H_residual computed at forward time (reference src/mhc/module.py:177-180).
    With the closure in the same graph inductor drops the copy (H unchanged) or orders the
    closure's read before the deferred write-back (H changed in place); a closure called
    outside the compiled region reads a materialised copy."""
    return H.clone(), w.new_empty((w.shape[0], 4))


class DynamicLayer(torch.autograd.Function):
    """Node A, dynamic fused weights: H -> (branch_input, w, link, post_link)."""

    @staticmethod
    def forward(ctx, H, phi, H_pre_base, H_post_base, H_res_base, alpha_pre, alpha_post, alpha_res,
                iters: int, eps: float):
        params = (phi, H_pre_base, H_post_base, H_res_base, alpha_pre, alpha_post, alpha_res)
        bi, x, w, aux = torch.ops.mhc.layer_dynamic_forward(H, *params, iters, eps)
        ctx.save_for_backward(H, x, w, aux, *params)
        ctx.iters = iters
        ctx.eps = eps
        ctx.set_materialize_grads(False)
        return (bi, w, *snapshot_links(H, w))

    @staticmethod
    def backward(ctx, d_bi, d_w, d_link, d_post):
        H, x, w, aux, *params = ctx.saved_tensors
        dH, gphi, gbias, galpha = torch.ops.mhc.layer_dynamic_backward(
            H, d_bi, d_link, d_post, *params, x, w, aux, ctx.iters, ctx.eps)
        return (dH, *_l._dynamic_param_grads(params, gphi, gbias, galpha), None, None)


class StaticLayer(torch.autograd.Function):
    """Node A, static weights: H -> (branch_input, w, link, post_link)."""

    @staticmethod
    def forward(ctx, H, H_pre_base, H_post_base, H_res_base, iters: int):
        params = (H_pre_base, H_post_base, H_res_base)
        bi, w = torch.ops.mhc.layer_static_forward(H, *params, iters)
        ctx.save_for_backward(H, w, *params)
        ctx.iters = iters
        ctx.set_materialize_grads(False)
        return (bi, w, *snapshot_links(H, w))

    @staticmethod
    def backward(ctx, d_bi, d_w, d_link, d_post):
        H, w, *params = ctx.saved_tensors
        dH, gbias = torch.ops.mhc.layer_static_backward(H, d_bi, d_link, d_post, *params, w, ctx.iters)
        return (dH, *_l._static_param_grads(params, gbias), None)


class PoolNode(torch.autograd.Function):
    """Sequence mean of the unfused dynamic layer, the node that writes dH:
    H -> (x [B,4D] f32, H_link, bi_link, w_link); the traced form of ``_layer._PoolNode``."""

    @staticmethod
    def forward(ctx, H):
        x = torch.ops.mhc.mean_pool(H)
        ctx.save_for_backward(H)
        ctx.set_materialize_grads(False)
        return (x, *_l._pool_links(H, x))

    @staticmethod
    def backward(ctx, gx, dH_new, d_bi, w):
        H, = ctx.saved_tensors
        if w is None:
            return None
        return torch.ops.mhc.layer_mix_dh(d_bi, dH_new, w, gx, H)


class GenericLayer(torch.autograd.Function):
    """Node A for weights produced by torch ops (the unfused dynamic path):
    (H_link, w, bi_link, w_link) -> (branch_input, w, link, post_link); the traced form of
    ``_layer._GenericLayer``."""

    @staticmethod
    def forward(ctx, H, w_in, bi_link, w_link):
        w = w_in.float()
        bi = torch.ops.mhc.layer_branch_input(H, w)
        ctx.save_for_backward(H, w)
        ctx.w_dtype = w_in.dtype
        ctx.set_materialize_grads(False)
        return (bi, w.clone() if w is w_in else w, *snapshot_links(H, w))

    @staticmethod
    def backward(ctx, d_bi, d_w, d_link, d_post):
        H, w = ctx.saved_tensors
        dpre, dres = torch.ops.mhc.layer_mix_reduce(H, d_bi, d_link, w)
        gw = torch.cat([dpre, torch.zeros_like(dpre) if d_post is None else d_post, dres], dim=1)
        if d_w is not None:
            gw = gw + d_w
        return d_link, gw.to(ctx.w_dtype), d_bi, w


class LayerAdd(torch.autograd.Function):
    """Node B, the closure: (link, branch_output, w, post_link) -> H_new.  Its backward returns
    dH_new as the link's gradient and dH_post [B,4] as post_link's, for node A to consume
    (neither is the true gradient of those inputs), and no gradient for w."""

    @staticmethod
    def forward(ctx, link, branch_output, w, post_link):
        ctx.save_for_backward(branch_output, w)
        ctx.h_dtype = link.dtype
        return torch.ops.mhc.layer_add_forward(link, branch_output, w)

    @staticmethod
    def backward(ctx, dH_new):
        bo, w = ctx.saved_tensors
        dH_new = dH_new.to(ctx.h_dtype)
        d_bo, dH_post = torch.ops.mhc.layer_add_backward(dH_new, bo, w)
        return dH_new, d_bo, None, dH_post


# --------------------------------------------------------------------------
# Stream expand / collapse (mhc.streams; no reference counterpart)
# --------------------------------------------------------------------------

@_op("stream_expand")
def stream_expand(x: Tensor, scale: float, dtype: Optional[torch.dtype] = None) -> Tensor:
    return _k.stream_expand(x, scale, dtype)


@stream_expand.register_fake
def _(x, scale, dtype=None):
    B, S, D = x.shape
    return x.new_empty(B, S, 4, D, dtype=dtype or x.dtype)


@_op("stream_collapse")
def stream_collapse(H: Tensor, scale: float, dtype: Optional[torch.dtype] = None) -> Tensor:
    return _k.stream_collapse(H, scale, dtype)


@stream_collapse.register_fake
def _(H, scale, dtype=None):
    B, S, _, D = H.shape
    return H.new_empty(B, S, D, dtype=dtype or H.dtype)


def _ends_setup(ctx, inputs, output):
    t, scale, _ = inputs
    ctx.scale = scale
    ctx.in_dtype = t.dtype


def _expand_bwd(ctx, dH):
    return torch.ops.mhc.stream_collapse(dH, ctx.scale, ctx.in_dtype), None, None


def _collapse_bwd(ctx, dy):
    return torch.ops.mhc.stream_expand(dy, ctx.scale, ctx.in_dtype), None, None


torch.library.register_autograd("mhc::stream_expand", _expand_bwd, setup_context=_ends_setup)
torch.library.register_autograd("mhc::stream_collapse", _collapse_bwd, setup_context=_ends_setup)
