"""HyperConnection module (reference src/mhc/module.py).

Same constructor arguments, parameter names / shapes / initialisation
(state_dict-compatible with the reference and with ``HyperConnectionTorch``),
and the same ``forward(H) -> (branch_input, add_residual)`` contract.  The
forward runs on the layer-level HIP path of ``_layer.py``.
"""

from __future__ import annotations

from typing import Callable, Tuple

import torch
import torch.nn as nn

from . import _layer, _library
from ._kernels import mean_pool
from .ops import fused_add_residual, fused_dynamic_weights, fused_stream_mix, sinkhorn_knopp


class HyperConnection(nn.Module):
    """Manifold-constrained hyper-connection over 4 residual streams.

    Args:
        dim: hidden dimension of each stream
        num_streams: number of streams (must be 4)
        layer_idx: layer index, selects the initial ``H_pre_base`` one-hot
        dynamic: compute input-dependent weights
        sinkhorn_iters: Sinkhorn-Knopp iterations for ``H_res``
        init_scale: initial value of the alpha / scale parameters
        eps: numerical-stability constant of the dynamic path
        use_fused_weights: use the fused Eq. 14-19 weights (else three Linears)

    Example::

        hc = HyperConnection(dim=512).cuda()
        H = torch.randn(2, 128, 4, 512, device="cuda")
        branch_input, add_residual = hc(H)
        H_new = add_residual(my_layer(branch_input))
    """

    def __init__(
        self,
        dim: int,
        num_streams: int = 4,
        layer_idx: int = 0,
        dynamic: bool = True,
        sinkhorn_iters: int = 20,
        init_scale: float = 0.1,
        eps: float = 1e-6,
        use_fused_weights: bool = True,
    ):
        super().__init__()
        if num_streams != 4:
            raise ValueError("HIP kernels require num_streams=4")
        self.dim = dim
        self.num_streams = num_streams
        self.dynamic = dynamic
        self.sinkhorn_iters = sinkhorn_iters
        self.init_scale = init_scale
        self.layer_idx = layer_idx
        self.eps = eps
        self.use_fused_weights = use_fused_weights and dynamic

        n = num_streams
        in_dim = n * dim
        out_dim = n * n + 2 * n

        self.H_post_base = nn.Parameter(torch.ones(n))
        pre = torch.zeros(n)
        pre[layer_idx % n] = 1.0
        self.H_pre_base = nn.Parameter(pre)
        self.H_res_base = nn.Parameter(torch.eye(n))

        if dynamic:
            if use_fused_weights:
                # phi [in_dim, 24], columns: H_pre (4), H_post (4), H_res (16, row-major)
                self.phi = nn.Parameter(torch.zeros(in_dim, out_dim))
                # 1-element tensors (FSDP / fully_shard friendly, as in the reference)
                self.alpha_pre = nn.Parameter(torch.tensor([init_scale]))
                self.alpha_post = nn.Parameter(torch.tensor([init_scale]))
                self.alpha_res = nn.Parameter(torch.tensor([init_scale]))
            else:
                self.W_post = nn.Linear(in_dim, n, bias=False)
                self.W_pre = nn.Linear(in_dim, n, bias=False)
                self.W_res = nn.Linear(in_dim, n * n, bias=False)
                nn.init.zeros_(self.W_post.weight)
                nn.init.zeros_(self.W_pre.weight)
                nn.init.zeros_(self.W_res.weight)
                self.scale_post = nn.Parameter(torch.tensor([init_scale]))
                self.scale_pre = nn.Parameter(torch.tensor([init_scale]))
                self.scale_res = nn.Parameter(torch.tensor([init_scale]))

    def _check_input(self, H: torch.Tensor) -> None:
        if H.dim() != 4 or H.shape[2] != self.num_streams or H.shape[3] != self.dim:
            raise ValueError(f"H must be (batch, seq, {self.num_streams}, {self.dim}), got {tuple(H.shape)}")

    def _unfused_weights(self, H: torch.Tensor, traced: bool = False) -> torch.Tensor:
        """Packed weights [B,24] of the unfused dynamic path from H (mean-pool included)."""
        pooled = torch.ops.mhc.mean_pool(H) if traced else _MeanPool.apply(H)
        return self._unfused_weights_from(pooled, traced)

    def _unfused_weights_from(self, pooled: torch.Tensor, traced: bool = False) -> torch.Tensor:
        """Packed weights [B,24] of the unfused dynamic path (reference src/mhc/module.py:141-163)
        from the sequence mean x [B,4D]: RMS-normalised x, three Linears, sigmoid (no x2 on
        H_post), normalisation with 1e-8 and Sinkhorn with eps 1e-8."""
        B = pooled.shape[0]
        n = self.num_streams
        x = pooled.to(self.W_pre.weight.dtype)
        rms = torch.sqrt((x * x).mean(dim=-1, keepdim=True) + self.eps)
        x = x / rms
        delta_post = self.W_post(x) * self.scale_post
        delta_pre = self.W_pre(x) * self.scale_pre
        delta_res = self.W_res(x).reshape(B, n, n) * self.scale_res
        H_post = torch.sigmoid(self.H_post_base + delta_post)
        H_pre = torch.sigmoid(self.H_pre_base + delta_pre)
        H_pre = H_pre / (H_pre.sum(dim=-1, keepdim=True) + 1e-8)
        M = (self.H_res_base + delta_res).contiguous()
        if traced:
            H_res = torch.ops.mhc.sinkhorn_forward(M, self.sinkhorn_iters, 1e-8)
        else:
            H_res = sinkhorn_knopp(M, self.sinkhorn_iters)
        return torch.cat([H_pre, H_post, H_res.reshape(B, n * n)], dim=1)

    def _compute_weights(self, H: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """(H_post [B,4], H_pre [B,4], H_res [B,4,4]), fp32 and differentiable, in the order
        of the reference's ``_compute_weights`` (reference src/mhc/module.py:103-163).

        ``forward`` derives the same weights inside the layer kernels and calls this method
        only when a subclass overrides it (then it composes the reference's way, see
        ``forward``).  It serves callers that inspect or log the mixing weights, on the same
        HIP ops (mean-pool, ``fused_dynamic_weights``, ``sinkhorn_knopp``).  The mean-pool is
        taken in fp32, as in ``forward``.
        """
        self._check_input(H)
        B = H.shape[0]
        n = self.num_streams
        traced = torch.compiler.is_compiling()
        if not self.dynamic:
            H_post = torch.sigmoid(self.H_post_base).unsqueeze(0).expand(B, -1)
            sg = torch.sigmoid(self.H_pre_base)
            H_pre = (sg / (sg.sum() + 1e-8)).unsqueeze(0).expand(B, -1)
            H_res = sinkhorn_knopp(self.H_res_base.unsqueeze(0).expand(B, -1, -1).contiguous(),
                                   self.sinkhorn_iters)
            return H_post.contiguous(), H_pre.contiguous(), H_res.contiguous()
        if self.use_fused_weights:
            x = torch.ops.mhc.mean_pool(H) if traced else _MeanPool.apply(H)
            bias = torch.cat([self.H_pre_base, self.H_post_base, self.H_res_base.flatten()])
            H_pre, H_post, H_res = fused_dynamic_weights(x, self.phi, bias, self.alpha_pre, self.alpha_post,
                                                         self.alpha_res, self.sinkhorn_iters, self.eps)
            return H_post, H_pre, H_res
        w = self._unfused_weights(H, traced=traced)
        return w[:, 4:8].contiguous(), w[:, 0:4].contiguous(), w[:, 8:].reshape(B, n, n).contiguous()

    def forward(self, H: torch.Tensor) -> Tuple[torch.Tensor, Callable[[torch.Tensor], torch.Tensor]]:
        """H (batch, seq, 4, dim) -> (branch_input (batch, seq, dim), add_residual).

        ``add_residual`` recomputes ``H_res @ H`` from ``H`` instead of keeping ``H_residual``
        (the reference's closure captures it, module.py:177-180).  In eager mode it therefore
        raises if ``H`` was modified in place between ``forward`` and the call, where the
        reference would still see the old values.  The check reads ``H``'s version counter,
        which every view of one storage shares: an in-place write to another slice of a buffer
        that ``H`` is a slice of also raises (pass a clone of the slice to avoid that).  Under
        torch.compile the closure reads a snapshot of ``H`` instead (the reference's
        semantics; inductor drops the copy when the closure runs in the same graph).  A strided
        ``H`` is made contiguous once, here, and that copy serves the forward, the closure and
        the backward.  An inference tensor (made under ``torch.inference_mode``) has no version
        counter, so for it the check does not run: modify such an ``H`` in place only after the
        closure has been called.

        A subclass that overrides ``_compute_weights`` gets the reference's composition on the
        HIP ops: its weights, ``fused_stream_mix`` and a closure over ``H_residual`` that calls
        ``fused_add_residual`` (module.py:165-182).
        """
        self._check_input(H)
        if type(self)._compute_weights is not HyperConnection._compute_weights:
            return self._forward_composed(H)
        H = H.contiguous()
        if torch.compiler.is_compiling():
            return self._forward_traced(H)
        # inference tensors (made under torch.inference_mode) keep no version counter
        version = None if H.is_inference() else H._version
        if not self.dynamic:
            bi, w, link, post_link = _layer._StaticLayer.apply(H, self.H_pre_base, self.H_post_base,
                                                               self.H_res_base, self.sinkhorn_iters)
        elif self.use_fused_weights:
            # a forward no gradient can reach (inference, or nothing requiring grad) keeps no pooled rows
            keep_x = torch.is_grad_enabled() and (H.requires_grad or any(p.requires_grad for p in (
                self.phi, self.H_pre_base, self.H_post_base, self.H_res_base, self.alpha_pre, self.alpha_post,
                self.alpha_res)))
            bi, w, link, post_link = _layer._DynamicLayer.apply(H, self.phi, self.H_pre_base, self.H_post_base,
                                                                self.H_res_base, self.alpha_pre, self.alpha_post,
                                                                self.alpha_res, self.sinkhorn_iters, self.eps,
                                                                keep_x)
        else:
            x, h_link, bi_link, w_link = _layer._PoolNode.apply(H)
            bi, w, link, post_link = _layer._GenericLayer.apply(h_link, self._unfused_weights_from(x), bi_link,
                                                                w_link)

        def add_residual(branch_output: torch.Tensor) -> torch.Tensor:
            if version is not None and H._version != version:
                raise RuntimeError(
                    "HyperConnection: H was modified in place after forward(H); add_residual recomputes "
                    "H_res @ H from H and would mix the modified values. Clone H before modifying it "
                    "(the version counter is shared by every view of H's storage).")
            return _layer._LayerAdd.apply(link, branch_output, w, post_link)

        return bi, add_residual

    def _forward_traced(self, H: torch.Tensor):
        """The same two nodes as ``forward``, on the torch.library ops; the closure reads a
        snapshot of the (contiguous) H."""
        if not self.dynamic:
            bi, w, link, post_link = _library.StaticLayer.apply(H, self.H_pre_base, self.H_post_base,
                                                                self.H_res_base, self.sinkhorn_iters)
        elif self.use_fused_weights:
            bi, w, link, post_link = _library.DynamicLayer.apply(H, self.phi, self.H_pre_base, self.H_post_base,
                                                                 self.H_res_base, self.alpha_pre, self.alpha_post,
                                                                 self.alpha_res, self.sinkhorn_iters, self.eps)
        else:
            x, h_link, bi_link, w_link = _library.PoolNode.apply(H)
            bi, w, link, post_link = _library.GenericLayer.apply(h_link, self._unfused_weights_from(x, True),
                                                                 bi_link, w_link)

        def add_residual(branch_output: torch.Tensor) -> torch.Tensor:
            return _library.LayerAdd.apply(link, branch_output, w, post_link)

        return bi, add_residual

    def _forward_composed(self, H: torch.Tensor):
        """The reference's forward (module.py:165-182) on the HIP ops, for subclasses that
        override ``_compute_weights``: the override's (H_post, H_pre, H_res), then
        ``fused_stream_mix``, and a closure over ``H_residual`` calling ``fused_add_residual``."""
        H_post, H_pre, H_res = self._compute_weights(H)
        branch_input, H_residual = fused_stream_mix(H.contiguous(), H_pre, H_res)

        def add_residual(branch_output: torch.Tensor) -> torch.Tensor:
            return fused_add_residual(H_residual, branch_output, H_post)

        return branch_input, add_residual

    def extra_repr(self) -> str:
        return (
            f"dim={self.dim}, num_streams={self.num_streams}, "
            f"dynamic={self.dynamic}, sinkhorn_iters={self.sinkhorn_iters}, "
            f"use_fused_weights={self.use_fused_weights}"
        )

    def init_weights(self, layer_idx=None):
        """Re-initialise every parameter, optionally moving to a new layer index
        (reference src/mhc/module.py:191-224)."""
        n = self.num_streams
        if layer_idx is not None:
            self.layer_idx = layer_idx
        nn.init.ones_(self.H_post_base)
        nn.init.zeros_(self.H_pre_base)
        with torch.no_grad():
            self.H_pre_base[self.layer_idx % n] = 1.0
        nn.init.eye_(self.H_res_base)
        if self.dynamic:
            if self.use_fused_weights:
                nn.init.zeros_(self.phi)
                nn.init.constant_(self.alpha_pre, self.init_scale)
                nn.init.constant_(self.alpha_post, self.init_scale)
                nn.init.constant_(self.alpha_res, self.init_scale)
            else:
                nn.init.zeros_(self.W_post.weight)
                nn.init.zeros_(self.W_pre.weight)
                nn.init.zeros_(self.W_res.weight)


class _MeanPool(torch.autograd.Function):
    """x = mean over the sequence, [B, 4*dim] f32, on the HIP mean-pool kernel.
    Backward is the broadcast grad_x / S (a stride-0 view, no copy)."""

    @staticmethod
    def forward(ctx, H):
        ctx.shape = H.shape
        ctx.dtype = H.dtype
        return mean_pool(H)

    @staticmethod
    def backward(ctx, gx):
        B, S, n, D = ctx.shape
        g = (gx / S).to(ctx.dtype).reshape(B, 1, n, D)
        return g.expand(B, S, n, D)
