"""Layer-level autograd for ``HyperConnection`` (reference src/mhc/module.py:103-182).

The reference composes ``H.mean`` -> ``fused_dynamic_weights`` ->
``fused_stream_mix`` and returns a closure over ``H_residual`` that calls
``fused_add_residual``.  Here the same math is split into two autograd nodes
that never materialise ``H_residual``:

* node A (``_DynamicLayer`` / ``_StaticLayer`` / ``_GenericLayer``):
  ``H -> (branch_input, w, link, post_link)`` where ``w`` [B,24] f32 packs
  H_pre (0:4), H_post (4:8) and H_res (8:24); ``link`` is a view of ``H`` and
  ``post_link`` an unwritten [B,4] tensor, both consumed only by the closure;
* node B (``_LayerAdd``, the closure): ``(link, branch_output, w, post_link)
  -> H_new``, recomputing ``H_res @ H`` on the fly.

Node B consumes the links, so the autograd engine runs node B's backward
before node A's.  Node B's backward computes ``d branch_output`` and
``dH_post`` and, instead of its true share of ``dH`` (which the engine would have
to add to node A's in another full pass), returns ``dH_new`` as the link's
gradient and ``dH_post`` as post_link's.  Node A's backward reads both and
writes the complete ``dH`` once.  The engine sums the closure's
gradients when it is called more than once, and a backward call that reaches
node B but not node A leaves no state behind.  The traced path (``_library.py``)
uses the same wiring on the ``torch.ops.mhc`` ops.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib


def _f32(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous() if t.dtype == torch.float32 else t.float().contiguous()


def _ws(lib, B, S, D, code, dev):
    return _lib.workspace(lib.mhc_layer_workspace_bytes(B, S, D, code), dev)


def _wsargs(ws):
    return (_lib.ptr(ws), 0 if ws is None else ws.numel())


def _grad_like(g: torch.Tensor, p: torch.Tensor) -> torch.Tensor:
    g = g.reshape(p.shape)
    return g if g.dtype == p.dtype else g.to(p.dtype)


def _in_h_dtype(t: Optional[torch.Tensor], H: torch.Tensor) -> Optional[torch.Tensor]:
    return None if t is None else t.contiguous().to(H.dtype)


# ---------------------------------------------------------------------------
# Launchers of the layer-level entry points.  Each allocates its outputs, calls
# the C ABI on torch's current stream and returns fresh tensors; the autograd
# nodes below and the torch.library ops (_library.py) are both built on them.
# ---------------------------------------------------------------------------

def dynamic_forward(H, phi, H_pre_base, H_post_base, H_res_base, alpha_pre, alpha_post, alpha_res,
                    iters: int, eps: float, keep_x: bool = True):
    """mhc_layer_dynamic_forward: H -> (branch_input, x [B,4D] f32, w [B,24] f32, aux [B,25] f32).
    Without keep_x (no backward follows) x is None and the pooled rows are not kept."""
    B, S, _, D = H.shape
    dev = _lib.require_gpu(H, phi)
    H = H.contiguous()
    params = [_f32(t) for t in (phi, H_pre_base, H_post_base, H_res_base,
                                alpha_pre.reshape(1), alpha_post.reshape(1), alpha_res.reshape(1))]
    bi = torch.empty(B, S, D, device=dev, dtype=H.dtype)
    x = torch.empty(B, 4 * D, device=dev, dtype=torch.float32) if keep_x else None
    w = torch.empty(B, 24, device=dev, dtype=torch.float32)
    aux = torch.empty(B, 25, device=dev, dtype=torch.float32)
    lib = _lib.load()
    code = _lib.dtype_code(H)
    ws = _ws(lib, B, S, D, code, dev)
    with _lib.on_device(dev):
        _lib.check(lib.mhc_layer_dynamic_forward(
            H.data_ptr(), code, *[p.data_ptr() for p in params], bi.data_ptr(), _lib.ptr(x), w.data_ptr(),
            aux.data_ptr(), B, S, D, int(iters), float(eps), *_wsargs(ws), _lib.stream(dev)),
            "layer_dynamic_forward")
    return bi, x, w, aux


def dynamic_backward(H, d_bi, dH_new, dH_post, phi, H_pre_base, H_post_base, H_res_base, alpha_pre,
                     alpha_post, alpha_res, x, w, aux, iters: int, eps: float, need_dH: bool = True):
    """mhc_layer_dynamic_backward -> (dH or None, grad_phi [4D,24], grad_bias [24], grad_alpha [3]), f32
    parameter gradients.  dH_new / dH_post are the closure's gradients (None if it was not called).
    x may be None at S = 1, where the pooled rows are H's rows and the kernels read them from H."""
    B, S, _, D = H.shape
    dev = _lib.require_gpu(H, phi)
    H = H.contiguous()
    d_bi = torch.zeros(B, S, D, device=dev, dtype=H.dtype) if d_bi is None else _in_h_dtype(d_bi, H)
    dH_new = _in_h_dtype(dH_new, H)
    dH_post = None if dH_post is None else _f32(dH_post)
    params = [_f32(t) for t in (phi, H_pre_base, H_post_base, H_res_base,
                                alpha_pre.reshape(1), alpha_post.reshape(1), alpha_res.reshape(1))]
    if x is None and S != 1:
        raise ValueError("mhc: layer_dynamic_backward needs the pooled rows x unless S == 1")
    x = None if x is None else _f32(x)
    w, aux = _f32(w), _f32(aux)
    dH = torch.empty_like(H) if need_dH else None
    gphi = torch.empty(4 * D, 24, device=dev, dtype=torch.float32)
    gbias = torch.empty(24, device=dev, dtype=torch.float32)
    galpha = torch.empty(3, device=dev, dtype=torch.float32)
    lib = _lib.load()
    code = _lib.dtype_code(H)
    ws = _ws(lib, B, S, D, code, dev)
    with _lib.on_device(dev):
        _lib.check(lib.mhc_layer_dynamic_backward(
            H.data_ptr(), code, d_bi.data_ptr(), _lib.ptr(dH_new), _lib.ptr(dH_post),
            *[p.data_ptr() for p in params], _lib.ptr(x), w.data_ptr(), aux.data_ptr(),
            _lib.ptr(dH), gphi.data_ptr(), gbias.data_ptr(), galpha.data_ptr(), B, S, D, int(iters), float(eps),
            *_wsargs(ws), _lib.stream(dev)), "layer_dynamic_backward")
    return dH, gphi, gbias, galpha


def static_forward(H, H_pre_base, H_post_base, H_res_base, iters: int):
    """mhc_layer_static_forward: H -> (branch_input, w [B,24] f32)."""
    B, S, _, D = H.shape
    dev = _lib.require_gpu(H, H_pre_base)
    H = H.contiguous()
    params = [_f32(t) for t in (H_pre_base, H_post_base, H_res_base)]
    bi = torch.empty(B, S, D, device=dev, dtype=H.dtype)
    w = torch.empty(B, 24, device=dev, dtype=torch.float32)
    lib = _lib.load()
    with _lib.on_device(dev):
        _lib.check(lib.mhc_layer_static_forward(
            H.data_ptr(), _lib.dtype_code(H), *[p.data_ptr() for p in params], bi.data_ptr(), w.data_ptr(),
            B, S, D, int(iters), _lib.stream(dev)), "layer_static_forward")
    return bi, w


def static_backward(H, d_bi, dH_new, dH_post, H_pre_base, H_post_base, H_res_base, w, iters: int,
                    need_dH: bool = True):
    """mhc_layer_static_backward -> (dH or None, grad_bias [24] f32: pre 0:4, post 4:8, res 8:24)."""
    B, S, _, D = H.shape
    dev = _lib.require_gpu(H, w)
    H = H.contiguous()
    d_bi = torch.zeros(B, S, D, device=dev, dtype=H.dtype) if d_bi is None else _in_h_dtype(d_bi, H)
    dH_new = _in_h_dtype(dH_new, H)
    dH_post = None if dH_post is None else _f32(dH_post)
    params = [_f32(t) for t in (H_pre_base, H_post_base, H_res_base)]
    w = _f32(w)
    dH = torch.empty_like(H) if need_dH else None
    gbias = torch.empty(24, device=dev, dtype=torch.float32)
    lib = _lib.load()
    code = _lib.dtype_code(H)
    ws = _ws(lib, B, S, D, code, dev)
    with _lib.on_device(dev):
        _lib.check(lib.mhc_layer_static_backward(
            H.data_ptr(), code, d_bi.data_ptr(), _lib.ptr(dH_new), _lib.ptr(dH_post),
            *[p.data_ptr() for p in params], w.data_ptr(), _lib.ptr(dH), gbias.data_ptr(), B, S, D,
            int(iters), *_wsargs(ws), _lib.stream(dev)), "layer_static_backward")
    return dH, gbias


def branch_input(H, w):
    """mhc_layer_branch_input: branch_input = sum_n w[:, n] H[n] with w [B,24] (H_pre in 0:4)."""
    B, S, _, D = H.shape
    dev = _lib.require_gpu(H, w)
    H = H.contiguous()
    w = _f32(w)
    bi = torch.empty(B, S, D, device=dev, dtype=H.dtype)
    lib = _lib.load()
    with _lib.on_device(dev):
        _lib.check(lib.mhc_layer_branch_input(H.data_ptr(), _lib.dtype_code(H), w.data_ptr(), bi.data_ptr(),
                                              B, S, D, _lib.stream(dev)), "layer_branch_input")
    return bi


def mix_backward(H, d_bi, dH_new, w, need_dH: bool = True):
    """mhc_layer_mix_backward -> (dH or None, dH_pre [B,4] f32, dH_res [B,16] f32)."""
    B, S, _, D = H.shape
    dev = _lib.require_gpu(H, w)
    H = H.contiguous()
    d_bi = torch.zeros(B, S, D, device=dev, dtype=H.dtype) if d_bi is None else _in_h_dtype(d_bi, H)
    dH_new = _in_h_dtype(dH_new, H)
    w = _f32(w)
    dH = torch.empty_like(H) if need_dH else None
    dpre = torch.empty(B, 4, device=dev, dtype=torch.float32)
    dres = torch.empty(B, 16, device=dev, dtype=torch.float32)
    lib = _lib.load()
    code = _lib.dtype_code(H)
    ws = _ws(lib, B, S, D, code, dev)
    with _lib.on_device(dev):
        _lib.check(lib.mhc_layer_mix_backward(
            H.data_ptr(), code, d_bi.data_ptr(), _lib.ptr(dH_new), w.data_ptr(), _lib.ptr(dH),
            dpre.data_ptr(), dres.data_ptr(), B, S, D, *_wsargs(ws), _lib.stream(dev)), "layer_mix_backward")
    return dH, dpre, dres


def mix_dh(d_bi, dH_new, w, grad_x, H_shape, h_dtype):
    """mhc_layer_mix_dh: dH = H_pre d_bi + H_res^T dH_new + grad_x / S in one pass, in h_dtype.
    d_bi / dH_new / grad_x may be None (no gradient reached them: zeros)."""
    B, S, _, D = H_shape
    dev = _lib.require_gpu(d_bi, dH_new, w, grad_x)
    d_bi = torch.zeros(B, S, D, device=dev, dtype=h_dtype) if d_bi is None else d_bi.contiguous().to(h_dtype)
    dH_new = None if dH_new is None else dH_new.contiguous().to(h_dtype)
    grad_x = torch.zeros(B, 4 * D, device=dev, dtype=torch.float32) if grad_x is None else _f32(grad_x)
    w = _f32(w)
    dH = torch.empty(B, S, 4, D, device=dev, dtype=h_dtype)
    lib = _lib.load()
    with _lib.on_device(dev):
        _lib.check(lib.mhc_layer_mix_dh(d_bi.data_ptr(), _lib.ptr(dH_new), _lib.dtype_code(dH), w.data_ptr(),
                                        grad_x.data_ptr(), dH.data_ptr(), B, S, D, _lib.stream(dev)),
                   "layer_mix_dh")
    return dH


def add_forward(H, branch_output, w):
    """mhc_layer_add_forward: H_new = H_res @ H + H_post * branch_output, in H's dtype."""
    B, S, _, D = H.shape
    if tuple(branch_output.shape) != (B, S, D):
        raise ValueError(f"branch_output must be ({B}, {S}, {D}), got {tuple(branch_output.shape)}")
    dev = _lib.require_gpu(H, branch_output, w)
    H = H.contiguous()
    bo = branch_output.contiguous()
    w = _f32(w)
    H_new = torch.empty_like(H)
    lib = _lib.load()
    with _lib.on_device(dev):
        _lib.check(lib.mhc_layer_add_forward(H.data_ptr(), _lib.dtype_code(H), bo.data_ptr(),
                                             _lib.dtype_code(bo), w.data_ptr(), H_new.data_ptr(), B, S, D,
                                             _lib.stream(dev)), "layer_add_forward")
    return H_new


def add_backward(dH_new, branch_output, w):
    """mhc_layer_add_backward -> (d_branch_output in branch_output's dtype, dH_post [B,4] f32)."""
    B, S, _, D = dH_new.shape
    dev = _lib.require_gpu(dH_new, branch_output, w)
    dH_new = dH_new.contiguous()
    bo = branch_output.contiguous()
    w = _f32(w)
    d_bo = torch.empty_like(bo)
    dH_post = torch.empty(B, 4, device=dev, dtype=torch.float32)
    lib = _lib.load()
    code = _lib.dtype_code(dH_new)
    ws = _ws(lib, B, S, D, code, dev)
    with _lib.on_device(dev):
        _lib.check(lib.mhc_layer_add_backward(dH_new.data_ptr(), code, bo.data_ptr(), _lib.dtype_code(bo),
                                              w.data_ptr(), d_bo.data_ptr(), dH_post.data_ptr(), B, S, D,
                                              *_wsargs(ws), _lib.stream(dev)), "layer_add_backward")
    return d_bo, dH_post


def _links(H: torch.Tensor, w: torch.Tensor):
    """The closure's two gradient carriers: a view of H (-> dH_new) and an unwritten [B, 4]
    tensor in w's dtype (-> dH_post).  The closure reads neither's values."""
    return H.view_as(H), w.new_empty((w.shape[0], 4))


class _DynamicLayer(torch.autograd.Function):
    """Node A, dynamic fused weights (module.py:119-139 + 177): H -> (branch_input, w, link, post_link)."""

    @staticmethod
    def forward(ctx, H, phi, H_pre_base, H_post_base, H_res_base, alpha_pre, alpha_post, alpha_res,
                iters: int, eps: float, keep_x: bool):
        params = (phi, H_pre_base, H_post_base, H_res_base, alpha_pre, alpha_post, alpha_res)
        # the pooled rows x serve only the backward: the caller drops them when no gradient can
        # reach this node (ctx.needs_input_grad reflects requires_grad even under torch.no_grad),
        # and at S = 1 they are H's rows, which the backward reads from H
        bi, x, w, aux = dynamic_forward(H, *params, iters, eps, keep_x=keep_x and H.shape[1] != 1)
        ctx.save_for_backward(H, x, w, aux, *params)
        ctx.iters = iters
        ctx.eps = eps
        ctx.set_materialize_grads(False)
        return (bi, w, *_links(H, w))

    @staticmethod
    def backward(ctx, d_bi, d_w, d_link, d_post):
        H, x, w, aux, *params = ctx.saved_tensors
        if x is None and H.shape[1] != 1:
            raise RuntimeError("mhc: backward through a dynamic layer forward that kept no pooled rows "
                               "(it ran where no gradient could reach it)")
        dH, gphi, gbias, galpha = dynamic_backward(H, d_bi, d_link, d_post, *params, x, w, aux,
                                                   ctx.iters, ctx.eps, need_dH=ctx.needs_input_grad[0])
        return (dH, *_dynamic_param_grads(params, gphi, gbias, galpha), None, None, None)


def _dynamic_param_grads(params, gphi, gbias, galpha):
    """The f32 kernel gradients reshaped and cast to each parameter."""
    return (_grad_like(gphi, params[0]), _grad_like(gbias[0:4], params[1]), _grad_like(gbias[4:8], params[2]),
            _grad_like(gbias[8:24], params[3]), _grad_like(galpha[0:1], params[4]),
            _grad_like(galpha[1:2], params[5]), _grad_like(galpha[2:3], params[6]))


def _static_param_grads(params, gbias):
    return (_grad_like(gbias[0:4], params[0]), _grad_like(gbias[4:8], params[1]),
            _grad_like(gbias[8:24], params[2]))


class _StaticLayer(torch.autograd.Function):
    """Node A, static weights (module.py:108-117 + 177): H -> (branch_input, w, link, post_link)."""

    @staticmethod
    def forward(ctx, H, H_pre_base, H_post_base, H_res_base, iters: int):
        params = (H_pre_base, H_post_base, H_res_base)
        bi, w = static_forward(H, *params, iters)
        ctx.save_for_backward(H, w, *params)
        ctx.iters = iters
        ctx.set_materialize_grads(False)
        return (bi, w, *_links(H, w))

    @staticmethod
    def backward(ctx, d_bi, d_w, d_link, d_post):
        H, w, *params = ctx.saved_tensors
        dH, gbias = static_backward(H, d_bi, d_link, d_post, *params, w, ctx.iters,
                                    need_dH=ctx.needs_input_grad[0])
        return (dH, *_static_param_grads(params, gbias), None)


def _pool_links(H: torch.Tensor, x: torch.Tensor):
    """The sequence-mean node's three gradient carriers: a view of H (-> dH_new), an unwritten
    [B,S,D] stride-0 tensor in H's dtype (-> d_branch_input) and an unwritten [B,24] f32 one
    (-> the weights w).  Node A reads none of their values."""
    B, S, _, D = H.shape
    return H.view_as(H), H.new_empty(()).expand(B, S, D), x.new_empty(()).expand(B, 24)


class _PoolNode(torch.autograd.Function):
    """Sequence mean of the unfused dynamic layer (module.py:123, 141-163), the node that writes dH:
    H -> (x [B,4D] f32, H_link, bi_link, w_link).

    x feeds the torch ops that make the weights; the links feed node A (``_GenericLayer``), whose
    backward returns dH_new, d_branch_input and w as their gradients.  The engine runs this node's
    backward after the weights' backward, so it holds grad_x too and writes
    dH = H_pre d_bi + H_res^T dH_new + grad_x / S in one pass, rounded once (mhc_layer_mix_dh),
    where a plain mean would have autograd add a broadcast grad_x / S into H.grad in two more."""

    @staticmethod
    def forward(ctx, H):
        from ._kernels import mean_pool

        x = mean_pool(H)
        ctx.shape = H.shape
        ctx.h_dtype = H.dtype
        ctx.set_materialize_grads(False)
        return (x, *_pool_links(H, x))

    @staticmethod
    def backward(ctx, gx, dH_new, d_bi, w):
        if w is None:  # node A's backward did not run in this call, so nothing reaches H
            return None
        return mix_dh(d_bi, dH_new, w, gx, ctx.shape, ctx.h_dtype)


class _GenericLayer(torch.autograd.Function):
    """Node A for weights produced by torch ops (the unfused dynamic path, module.py:141-163):
    (H_link, w, bi_link, w_link) -> (branch_input, w, link, post_link), differentiable in w.

    H_link, bi_link and w_link come from ``_PoolNode``.  The backward runs the reductions only
    (dH_pre, dH_res) and hands dH_new, d_branch_input and w to the pool node as the links'
    gradients; that node writes dH once grad_x is known."""

    @staticmethod
    def forward(ctx, H, w_in, bi_link, w_link):
        w = _f32(w_in)
        bi = branch_input(H, w)
        ctx.save_for_backward(H, w)
        ctx.w_dtype = w_in.dtype
        ctx.set_materialize_grads(False)
        return (bi, w.clone() if w is w_in else w, *_links(H, w))

    @staticmethod
    def backward(ctx, d_bi, d_w, d_link, d_post):
        H, w = ctx.saved_tensors
        _, dpre, dres = mix_backward(H, d_bi, d_link, w, need_dH=False)
        gw = torch.cat([dpre, torch.zeros_like(dpre) if d_post is None else d_post, dres], dim=1)
        if d_w is not None:
            gw = gw + d_w
        to_pool = ctx.needs_input_grad[0]
        return ((d_link if to_pool else None), gw.to(ctx.w_dtype), (d_bi if to_pool else None),
                (w if to_pool else None))


class _LayerAdd(torch.autograd.Function):
    """Node B, the closure: (link, branch_output, w, post_link) -> H_new = H_res @ H +
    H_post * branch_output (module.py:179-180 with H_residual recomputed from H).

    Its backward returns dH_new as the link's gradient and dH_post [B,4] as post_link's.
    Neither is the true gradient of that input: both only reach node A, which folds dH_new
    into dH (one pass) and dH_post into the H_post weight gradients.  It returns no gradient
    for w.  A backward call that reaches node B but not node A leaves nothing behind."""

    @staticmethod
    def forward(ctx, link, branch_output, w, post_link):
        H_new = add_forward(link, branch_output, w)
        ctx.save_for_backward(branch_output, w)
        ctx.h_dtype = link.dtype
        return H_new

    @staticmethod
    def backward(ctx, dH_new):
        bo, w = ctx.saved_tensors
        dH_new = dH_new.contiguous().to(ctx.h_dtype)
        d_bo, dH_post = add_backward(dH_new, bo, w)
        return ((dH_new if ctx.needs_input_grad[0] else None), d_bo, None,
                (dH_post if ctx.needs_input_grad[3] else None))
