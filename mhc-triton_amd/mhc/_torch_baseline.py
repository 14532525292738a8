"""Pure-PyTorch implementations of the mHC ops (public ``*_torch`` API).

Same math, signatures and parameter layout as the reference's
src/mhc/_torch_baseline.py, written with plain torch ops so they run on any
device (CPU included) and differentiate through autograd.  They are the
"PyTorch" column of benchmarks; the HIP path never calls them.
"""

from __future__ import annotations

from typing import Callable, Tuple

import torch
import torch.nn as nn


def sinkhorn_knopp_torch(M: torch.Tensor, num_iters: int = 20, eps: float = 1e-8) -> torch.Tensor:
    """Doubly-stochastic projection of (..., 4, 4) matrices
    (reference _torch_baseline.py:12-35): P = |M| + eps, then ``num_iters``
    rounds of row and column normalisation, each sum offset by eps."""
    P = M.abs() + eps
    for _ in range(num_iters):
        P = P / (P.sum(dim=-1, keepdim=True) + eps)
        P = P / (P.sum(dim=-2, keepdim=True) + eps)
    return P


def _split24(t: torch.Tensor):
    return t[..., 0:4], t[..., 4:8], t[..., 8:24]


def fused_dynamic_weights_torch(
    x: torch.Tensor,
    phi: torch.Tensor,
    bias: torch.Tensor,
    alpha_pre: torch.Tensor,
    alpha_post: torch.Tensor,
    alpha_res: torch.Tensor,
    sinkhorn_iters: int = 20,
    eps: float = 1e-6,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Eq. 14-19 (reference _torch_baseline.py:38-111).

    raw = x @ phi; inv_rms = 1/sqrt(sum(x^2)/in_dim + eps);
    s = inv_rms * alpha * raw + bias (groups pre 0:4, post 4:8, res 8:24);
    H_pre = sigmoid(s_pre)/(sum + eps), H_post = 2 sigmoid(s_post),
    H_res = Sinkhorn(s_res as 4x4, sinkhorn_iters, eps).
    """
    batch, in_dim = x.shape
    raw = x @ phi
    inv_rms = 1.0 / torch.sqrt((x * x).sum(dim=-1, keepdim=True) / in_dim + eps)
    r_pre, r_post, r_res = _split24(raw)
    b_pre, b_post, b_res = _split24(bias)
    s_pre = inv_rms * alpha_pre * r_pre + b_pre
    s_post = inv_rms * alpha_post * r_post + b_post
    s_res = inv_rms * alpha_res * r_res + b_res
    sig = torch.sigmoid(s_pre)
    H_pre = sig / (sig.sum(dim=-1, keepdim=True) + eps)
    H_post = 2.0 * torch.sigmoid(s_post)
    H_res = sinkhorn_knopp_torch(s_res.reshape(batch, 4, 4), sinkhorn_iters, eps)
    return H_pre, H_post, H_res


def fused_stream_mix_torch(H: torch.Tensor, H_pre: torch.Tensor, H_res: torch.Tensor
                           ) -> Tuple[torch.Tensor, torch.Tensor]:
    """branch_input = sum_n H_pre[b,n] H[b,s,n,:]; H_residual[n] = sum_m H_res[b,n,m] H[b,s,m,:]
    (reference _torch_baseline.py:114-143)."""
    branch_input = torch.einsum("bn,bsnd->bsd", H_pre, H)
    H_residual = torch.einsum("bnm,bsmd->bsnd", H_res, H)
    return branch_input, H_residual


def fused_add_residual_torch(H_residual: torch.Tensor, branch_output: torch.Tensor, H_post: torch.Tensor
                             ) -> torch.Tensor:
    """H_new[b,s,n,:] = H_residual[b,s,n,:] + H_post[b,n] * branch_output[b,s,:]
    (reference _torch_baseline.py:146-166)."""
    return H_residual + H_post[:, None, :, None] * branch_output[:, :, None, :]


class HyperConnectionTorch(nn.Module):
    """Pure-PyTorch HyperConnection (reference _torch_baseline.py:169-336); same
    parameters as ``HyperConnection`` so state dicts load across the two."""

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
            raise ValueError("num_streams must be 4 for compatibility")
        self.dim = dim
        self.num_streams = num_streams
        self.dynamic = dynamic
        self.sinkhorn_iters = sinkhorn_iters
        self.layer_idx = layer_idx
        self.eps = eps
        self.use_fused_weights = use_fused_weights and dynamic
        n = num_streams
        in_dim, out_dim = n * dim, n * n + 2 * n
        self.H_post_base = nn.Parameter(torch.ones(n))
        pre = torch.zeros(n)
        pre[layer_idx % n] = 1.0
        self.H_pre_base = nn.Parameter(pre)
        self.H_res_base = nn.Parameter(torch.eye(n))
        if dynamic:
            if use_fused_weights:
                self.phi = nn.Parameter(torch.zeros(in_dim, out_dim))
                self.alpha_pre = nn.Parameter(torch.tensor([init_scale]))
                self.alpha_post = nn.Parameter(torch.tensor([init_scale]))
                self.alpha_res = nn.Parameter(torch.tensor([init_scale]))
            else:
                self.W_post = nn.Linear(in_dim, n, bias=False)
                self.W_pre = nn.Linear(in_dim, n, bias=False)
                self.W_res = nn.Linear(in_dim, n * n, bias=False)
                for lin in (self.W_post, self.W_pre, self.W_res):
                    nn.init.zeros_(lin.weight)
                self.scale_post = nn.Parameter(torch.tensor([init_scale]))
                self.scale_pre = nn.Parameter(torch.tensor([init_scale]))
                self.scale_res = nn.Parameter(torch.tensor([init_scale]))

    def _compute_weights(self, H: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """(H_post, H_pre, H_res) -- note the order (reference
        _torch_baseline.py:227-286)."""
        n = self.num_streams
        batch = H.shape[0]
        if not self.dynamic:
            H_post = torch.sigmoid(self.H_post_base).unsqueeze(0).expand(batch, -1)
            sig = torch.sigmoid(self.H_pre_base)
            H_pre = (sig / (sig.sum() + 1e-8)).unsqueeze(0).expand(batch, -1)
            H_res = sinkhorn_knopp_torch(self.H_res_base.unsqueeze(0).expand(batch, -1, -1).contiguous(),
                                         self.sinkhorn_iters)
            return H_post.contiguous(), H_pre.contiguous(), H_res.contiguous()
        x = H.mean(dim=1).reshape(batch, n * self.dim)
        if self.use_fused_weights:
            bias = torch.cat([self.H_pre_base, self.H_post_base, self.H_res_base.flatten()])
            H_pre, H_post, H_res = fused_dynamic_weights_torch(
                x, self.phi, bias, self.alpha_pre, self.alpha_post, self.alpha_res, self.sinkhorn_iters, self.eps)
            return H_post.contiguous(), H_pre.contiguous(), H_res.contiguous()
        x = x / torch.sqrt((x * x).mean(dim=-1, keepdim=True) + self.eps)
        H_post = torch.sigmoid(self.H_post_base + self.W_post(x) * self.scale_post)
        sig = torch.sigmoid(self.H_pre_base + self.W_pre(x) * self.scale_pre)
        H_pre = sig / (sig.sum(dim=-1, keepdim=True) + 1e-8)
        H_res = sinkhorn_knopp_torch(
            (self.H_res_base + self.W_res(x).reshape(batch, n, n) * self.scale_res).contiguous(),
            self.sinkhorn_iters)
        return H_post.contiguous(), H_pre.contiguous(), H_res.contiguous()

    def forward(self, H: torch.Tensor) -> Tuple[torch.Tensor, Callable[[torch.Tensor], torch.Tensor]]:
        H_post, H_pre, H_res = self._compute_weights(H)
        branch_input, H_residual = fused_stream_mix_torch(H, H_pre, H_res)

        def add_residual(branch_output: torch.Tensor) -> torch.Tensor:
            return fused_add_residual_torch(H_residual, branch_output, H_post)

        return branch_input, add_residual

    def extra_repr(self) -> str:
        return (
            f"dim={self.dim}, num_streams={self.num_streams}, "
            f"dynamic={self.dynamic}, sinkhorn_iters={self.sinkhorn_iters}, "
            f"use_fused_weights={self.use_fused_weights}"
        )
