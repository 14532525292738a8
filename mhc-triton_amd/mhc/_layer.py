"""Layer-level autograd for ``HyperConnection`` (reference src/mhc/module.py:103-182).

The reference composes ``H.mean`` -> ``fused_dynamic_weights`` ->
``fused_stream_mix`` and returns a closure over ``H_residual`` that calls
``fused_add_residual``.  Here the same math is split into two autograd nodes
that never materialise ``H_residual``:

* node A (``_DynamicLayer`` / ``_StaticLayer`` / ``_GenericLayer``):
  ``H -> (branch_input, w)`` where ``w`` [B,24] f32 packs H_pre (0:4),
  H_post (4:8) and H_res (8:24);
* node B (``_LayerAdd``, the closure): ``(H, branch_output, w) -> H_new``,
  recomputing ``H_res @ H`` on the fly.

Node B consumes ``w``, so the autograd engine runs node B's backward before
node A's.  Node B's backward computes ``d branch_output`` and ``dH_post`` and,
instead of returning its share of ``dH`` (which the engine would have to add to
node A's in another full pass), hands ``dH_new`` and ``dH_post`` to node A
through a shared ``_Stash``; node A then writes the complete ``dH`` once.
Node B returns no gradient for ``H`` or ``w``.
"""

from __future__ import annotations

from typing import List, Optional, Tuple

import torch

from . import _lib


class _Stash:
    """Per-forward-call channel from node B's backward to node A's backward."""

    __slots__ = ("items",)

    def __init__(self):
        self.items: List[Tuple[torch.Tensor, torch.Tensor]] = []

    def put(self, dH_new: torch.Tensor, dH_post: torch.Tensor) -> None:
        self.items.append((dH_new, dH_post))

    def take(self) -> Tuple[Optional[torch.Tensor], Optional[torch.Tensor]]:
        items, self.items = self.items, []
        if not items:
            return None, None
        dH_new, dH_post = items[0]
        for a, b in items[1:]:  # the closure was called more than once
            dH_new = dH_new + a
            dH_post = dH_post + b
        return dH_new, dH_post


def _f32(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous() if t.dtype == torch.float32 else t.float().contiguous()


def _ws(lib, B, S, D, code, dev):
    return _lib.workspace(lib.mhc_layer_workspace_bytes(B, S, D, code), dev)


def _wsargs(ws):
    return (_lib.ptr(ws), 0 if ws is None else ws.numel())


def _grad_like(g: torch.Tensor, p: torch.Tensor) -> torch.Tensor:
    g = g.reshape(p.shape)
    return g if g.dtype == p.dtype else g.to(p.dtype)


class _DynamicLayer(torch.autograd.Function):
    """Node A, dynamic fused weights (module.py:119-139 + 177)."""

    @staticmethod
    def forward(ctx, H, phi, H_pre_base, H_post_base, H_res_base, alpha_pre, alpha_post, alpha_res,
                stash: _Stash, iters: int, eps: float):
        B, S, _, D = H.shape
        dev = _lib.require_gpu(H, phi)
        H = H.contiguous()
        params = [_f32(t) for t in (phi, H_pre_base, H_post_base, H_res_base,
                                    alpha_pre.reshape(1), alpha_post.reshape(1), alpha_res.reshape(1))]
        bi = torch.empty(B, S, D, device=dev, dtype=H.dtype)
        x = torch.empty(B, 4 * D, device=dev, dtype=torch.float32)
        w = torch.empty(B, 24, device=dev, dtype=torch.float32)
        aux = torch.empty(B, 25, device=dev, dtype=torch.float32)
        lib = _lib.load()
        code = _lib.dtype_code(H)
        ws = _ws(lib, B, S, D, code, dev)
        with _lib.on_device(dev):
            _lib.check(lib.mhc_layer_dynamic_forward(
                H.data_ptr(), code, *[p.data_ptr() for p in params], bi.data_ptr(), x.data_ptr(), w.data_ptr(),
                aux.data_ptr(), B, S, D, int(iters), float(eps), *_wsargs(ws), _lib.stream(dev)),
                "layer_dynamic_forward")
        ctx.save_for_backward(H, x, w, aux, *params)
        ctx.stash = stash
        ctx.iters = iters
        ctx.eps = eps
        ctx.param_refs = (phi, H_pre_base, H_post_base, H_res_base, alpha_pre, alpha_post, alpha_res)
        ctx.set_materialize_grads(False)
        return bi, w

    @staticmethod
    def backward(ctx, d_bi, d_w):
        H, x, w, aux, *params = ctx.saved_tensors
        refs = ctx.param_refs
        B, S, _, D = H.shape
        dev = H.device
        dH_new, dH_post = ctx.stash.take()
        if d_bi is None:
            d_bi = torch.zeros(B, S, D, device=dev, dtype=H.dtype)
        d_bi = d_bi.contiguous().to(H.dtype)
        if dH_new is not None:
            dH_new = dH_new.contiguous().to(H.dtype)
        need_dH = ctx.needs_input_grad[0]
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
                *[p.data_ptr() for p in params], x.data_ptr(), w.data_ptr(), aux.data_ptr(), _lib.ptr(dH),
                gphi.data_ptr(), gbias.data_ptr(), galpha.data_ptr(), B, S, D, int(ctx.iters), float(ctx.eps),
                *_wsargs(ws), _lib.stream(dev)), "layer_dynamic_backward")
        return (dH, _grad_like(gphi, refs[0]), _grad_like(gbias[0:4], refs[1]), _grad_like(gbias[4:8], refs[2]),
                _grad_like(gbias[8:24], refs[3]), _grad_like(galpha[0:1], refs[4]),
                _grad_like(galpha[1:2], refs[5]), _grad_like(galpha[2:3], refs[6]), None, None, None)


class _StaticLayer(torch.autograd.Function):
    """Node A, static weights (module.py:108-117 + 177)."""

    @staticmethod
    def forward(ctx, H, H_pre_base, H_post_base, H_res_base, stash: _Stash, iters: int):
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
        ctx.save_for_backward(H, w, *params)
        ctx.stash = stash
        ctx.iters = iters
        ctx.param_refs = (H_pre_base, H_post_base, H_res_base)
        ctx.set_materialize_grads(False)
        return bi, w

    @staticmethod
    def backward(ctx, d_bi, d_w):
        H, w, *params = ctx.saved_tensors
        refs = ctx.param_refs
        B, S, _, D = H.shape
        dev = H.device
        dH_new, dH_post = ctx.stash.take()
        if d_bi is None:
            d_bi = torch.zeros(B, S, D, device=dev, dtype=H.dtype)
        d_bi = d_bi.contiguous().to(H.dtype)
        if dH_new is not None:
            dH_new = dH_new.contiguous().to(H.dtype)
        dH = torch.empty_like(H) if ctx.needs_input_grad[0] else None
        gbias = torch.empty(24, device=dev, dtype=torch.float32)
        lib = _lib.load()
        code = _lib.dtype_code(H)
        ws = _ws(lib, B, S, D, code, dev)
        with _lib.on_device(dev):
            _lib.check(lib.mhc_layer_static_backward(
                H.data_ptr(), code, d_bi.data_ptr(), _lib.ptr(dH_new), _lib.ptr(dH_post),
                *[p.data_ptr() for p in params], w.data_ptr(), _lib.ptr(dH), gbias.data_ptr(), B, S, D,
                int(ctx.iters), *_wsargs(ws), _lib.stream(dev)), "layer_static_backward")
        return (dH, _grad_like(gbias[0:4], refs[0]), _grad_like(gbias[4:8], refs[1]),
                _grad_like(gbias[8:24], refs[2]), None, None)


class _GenericLayer(torch.autograd.Function):
    """Node A for weights produced by torch ops (the unfused dynamic path,
    module.py:141-163): (H, w) -> (branch_input, w), differentiable in w."""

    @staticmethod
    def forward(ctx, H, w_in, stash: _Stash):
        B, S, _, D = H.shape
        dev = _lib.require_gpu(H, w_in)
        H = H.contiguous()
        w = _f32(w_in)
        bi = torch.empty(B, S, D, device=dev, dtype=H.dtype)
        lib = _lib.load()
        with _lib.on_device(dev):
            _lib.check(lib.mhc_layer_branch_input(H.data_ptr(), _lib.dtype_code(H), w.data_ptr(), bi.data_ptr(),
                                                  B, S, D, _lib.stream(dev)), "layer_branch_input")
        ctx.save_for_backward(H, w)
        ctx.stash = stash
        ctx.w_dtype = w_in.dtype
        ctx.set_materialize_grads(False)
        return bi, w

    @staticmethod
    def backward(ctx, d_bi, d_w):
        H, w = ctx.saved_tensors
        B, S, _, D = H.shape
        dev = H.device
        dH_new, dH_post = ctx.stash.take()
        if d_bi is None:
            d_bi = torch.zeros(B, S, D, device=dev, dtype=H.dtype)
        d_bi = d_bi.contiguous().to(H.dtype)
        if dH_new is not None:
            dH_new = dH_new.contiguous().to(H.dtype)
        dH = torch.empty_like(H) if ctx.needs_input_grad[0] else None
        gw = torch.zeros(B, 24, device=dev, dtype=torch.float32)
        dpre = torch.empty(B, 4, device=dev, dtype=torch.float32)
        dres = torch.empty(B, 16, device=dev, dtype=torch.float32)
        lib = _lib.load()
        code = _lib.dtype_code(H)
        ws = _ws(lib, B, S, D, code, dev)
        with _lib.on_device(dev):
            _lib.check(lib.mhc_layer_mix_backward(
                H.data_ptr(), code, d_bi.data_ptr(), _lib.ptr(dH_new), w.data_ptr(), _lib.ptr(dH),
                dpre.data_ptr(), dres.data_ptr(), B, S, D, *_wsargs(ws), _lib.stream(dev)), "layer_mix_backward")
        gw[:, 0:4] = dpre
        gw[:, 8:24] = dres
        if dH_post is not None:
            gw[:, 4:8] = dH_post
        if d_w is not None:
            gw = gw + d_w
        return dH, gw.to(ctx.w_dtype), None


class _LayerAdd(torch.autograd.Function):
    """Node B, the closure: H_new = H_res @ H + H_post * branch_output
    (module.py:179-180 with H_residual recomputed from H)."""

    @staticmethod
    def forward(ctx, H, branch_output, w, stash: _Stash):
        B, S, _, D = H.shape
        if tuple(branch_output.shape) != (B, S, D):
            raise ValueError(f"branch_output must be ({B}, {S}, {D}), got {tuple(branch_output.shape)}")
        dev = _lib.require_gpu(H, branch_output, w)
        H = H.contiguous()
        bo = branch_output.contiguous()
        H_new = torch.empty_like(H)
        lib = _lib.load()
        with _lib.on_device(dev):
            _lib.check(lib.mhc_layer_add_forward(H.data_ptr(), _lib.dtype_code(H), bo.data_ptr(),
                                                 _lib.dtype_code(bo), w.data_ptr(), H_new.data_ptr(), B, S, D,
                                                 _lib.stream(dev)), "layer_add_forward")
        ctx.save_for_backward(bo, w)
        ctx.stash = stash
        ctx.shape = (B, S, D)
        ctx.h_dtype = H.dtype
        return H_new

    @staticmethod
    def backward(ctx, dH_new):
        bo, w = ctx.saved_tensors
        B, S, D = ctx.shape
        dev = bo.device
        dH_new = dH_new.contiguous().to(ctx.h_dtype)
        d_bo = torch.empty_like(bo)
        dH_post = torch.empty(B, 4, device=dev, dtype=torch.float32)
        lib = _lib.load()
        code = _lib.dtype_code(dH_new)
        ws = _ws(lib, B, S, D, code, dev)
        with _lib.on_device(dev):
            _lib.check(lib.mhc_layer_add_backward(dH_new.data_ptr(), code, bo.data_ptr(), _lib.dtype_code(bo),
                                                  w.data_ptr(), d_bo.data_ptr(), dH_post.data_ptr(), B, S, D,
                                                  *_wsargs(ws), _lib.stream(dev)), "layer_add_backward")
        if ctx.needs_input_grad[2]:
            ctx.stash.put(dH_new, dH_post)
        return None, d_bo, None, None
