"""Torch restatement of the reference's pure-PyTorch layer.  TEST INFRASTRUCTURE ONLY.

Used by tests/ (torch autograd of this forward is an independent check of the
hand-derived gradients in mhc_oracle.py) and by bench.py's ``cpu_baseline`` leg
(the reference's CPU PyTorch path, timed on the host cores).  It restates
src/mhc/_torch_baseline.py:12-166 and the module wiring of
_torch_baseline.py:227-336 as functions over a parameter dict; bulk inputs are
upcast to ``dtype`` (fp32 by default) because the reference's own path raises on
a bf16 H with fp32 weights.
"""

from __future__ import annotations

import torch


def sinkhorn(M, iters=20, eps=1e-8):
    P = M.abs() + eps
    for _ in range(iters):
        P = P / (P.sum(dim=-1, keepdim=True) + eps)
        P = P / (P.sum(dim=-2, keepdim=True) + eps)
    return P


def dynamic_weights(x, phi, bias, a_pre, a_post, a_res, iters=20, eps=1e-6):
    R, K = x.shape
    raw = x @ phi
    inv_rms = 1.0 / torch.sqrt((x * x).sum(dim=-1, keepdim=True) / K + eps)
    s_pre = inv_rms * a_pre * raw[:, 0:4] + bias[0:4]
    s_post = inv_rms * a_post * raw[:, 4:8] + bias[4:8]
    s_res = inv_rms * a_res * raw[:, 8:24] + bias[8:24]
    sg = torch.sigmoid(s_pre)
    H_pre = sg / (sg.sum(dim=-1, keepdim=True) + eps)
    H_post = 2.0 * torch.sigmoid(s_post)
    H_res = sinkhorn(s_res.reshape(R, 4, 4), iters, eps)
    return H_pre, H_post, H_res


def stream_mix(H, H_pre, H_res):
    return torch.einsum("bn,bsnd->bsd", H_pre, H), torch.einsum("bnm,bsmd->bsnd", H_res, H)


def add_residual(H_residual, bo, H_post):
    return H_residual + H_post[:, None, :, None] * bo[:, :, None, :]


def layer_weights(p, H, dynamic=True, fused=True, iters=20, eps=1e-6):
    """(H_post, H_pre, H_res) for a parameter dict p (module parameter names)."""
    B, S, n, D = H.shape
    if not dynamic:
        H_post = torch.sigmoid(p["H_post_base"]).unsqueeze(0).expand(B, -1)
        sg = torch.sigmoid(p["H_pre_base"])
        H_pre = (sg / (sg.sum() + 1e-8)).unsqueeze(0).expand(B, -1)
        H_res = sinkhorn(p["H_res_base"].unsqueeze(0).expand(B, -1, -1), iters, 1e-8)
        return H_post, H_pre, H_res
    x = H.mean(dim=1).reshape(B, n * D)
    if fused:
        bias = torch.cat([p["H_pre_base"], p["H_post_base"], p["H_res_base"].flatten()])
        H_pre, H_post, H_res = dynamic_weights(x, p["phi"], bias, p["alpha_pre"], p["alpha_post"], p["alpha_res"],
                                               iters, eps)
        return H_post, H_pre, H_res
    x = x / torch.sqrt((x * x).mean(dim=-1, keepdim=True) + eps)
    H_post = torch.sigmoid(p["H_post_base"] + (x @ p["W_post.weight"].T) * p["scale_post"])
    sg = torch.sigmoid(p["H_pre_base"] + (x @ p["W_pre.weight"].T) * p["scale_pre"])
    H_pre = sg / (sg.sum(dim=-1, keepdim=True) + 1e-8)
    H_res = sinkhorn(p["H_res_base"] + (x @ p["W_res.weight"].T).reshape(B, 4, 4) * p["scale_res"], iters, 1e-8)
    return H_post, H_pre, H_res


def layer_forward(p, H, bo, dynamic=True, fused=True, iters=20, eps=1e-6, dtype=torch.float32):
    """(branch_input, H_new) with every tensor upcast to `dtype`."""
    H = H.to(dtype)
    bo = bo.to(dtype)
    p = {k: v.to(dtype) for k, v in p.items()}
    H_post, H_pre, H_res = layer_weights(p, H, dynamic, fused, iters, eps)
    bi, hr = stream_mix(H, H_pre, H_res)
    return bi, add_residual(hr, bo, H_post)


def layer_grads(p, H, bo, dH_new, d_bi, dynamic=True, fused=True, iters=20, eps=1e-6, dtype=torch.float32):
    """Forward + torch autograd backward; returns (bi, H_new, grads dict)."""
    leaves = {k: v.detach().to(dtype).clone().requires_grad_(True) for k, v in p.items()}
    Hl = H.detach().to(dtype).clone().requires_grad_(True)
    bol = bo.detach().to(dtype).clone().requires_grad_(True)
    bi, H_new = layer_forward(leaves, Hl, bol, dynamic, fused, iters, eps, dtype)
    torch.autograd.backward([H_new, bi], [dH_new.to(dtype), d_bi.to(dtype)])
    g = {k: v.grad for k, v in leaves.items()}
    g["H"] = Hl.grad
    g["bo"] = bol.grad
    return bi.detach(), H_new.detach(), g
