"""Forward launchers over the gfx950 HIP kernels.

Same names, arguments and output dtypes as the reference's launcher layer
(src/mhc/_kernels.py:597-752); each call goes through the C ABI of
``libmhc_hip.so``.  ``block_dim`` (a Triton tile size in the reference) is
accepted for compatibility and ignored: the HIP kernels pick their own tiling.
"""

from __future__ import annotations

from typing import Tuple, Union

import torch

from . import _lib


class ShapeError(AssertionError, ValueError):
    """Bad argument shape.  Subclasses AssertionError like the reference's
    ``assert`` checks (src/mhc/_kernels.py:609,634,671,726-727) and ValueError."""


def _f32(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous() if t.dtype == torch.float32 else t.float().contiguous()


def _alpha_tensor(a, dev) -> torch.Tensor:
    if isinstance(a, torch.Tensor):
        if a.numel() != 1:
            raise ShapeError(f"alpha must have one element, got shape {tuple(a.shape)}")
        return _f32(a.reshape(1).to(dev))
    return torch.tensor([float(a)], dtype=torch.float32, device=dev)


def sinkhorn_forward(M: torch.Tensor, num_iters: int = 20, eps: float = 1e-8) -> torch.Tensor:
    """Sinkhorn-Knopp projection of a batch of 4x4 matrices (reference
    src/mhc/_kernels.py:597-614).  Returns a new tensor in M's dtype."""
    if M.dim() < 2 or tuple(M.shape[-2:]) != (4, 4):
        raise ShapeError("Expected (..., 4, 4)")
    if num_iters < 0:
        raise ValueError("num_iters must be >= 0")
    dev = _lib.require_gpu(M)
    M = M.contiguous()
    out = torch.empty_like(M)
    lib = _lib.load()
    with _lib.on_device(dev):
        _lib.check(lib.mhc_sinkhorn_forward(M.data_ptr(), out.data_ptr(), M.numel() // 16, _lib.dtype_code(M),
                                            int(num_iters), float(eps), _lib.stream(dev)), "sinkhorn_forward")
    return out


def stream_mix_forward(H: torch.Tensor, H_pre: torch.Tensor, H_res: torch.Tensor,
                       block_dim: int = 128) -> Tuple[torch.Tensor, torch.Tensor]:
    """branch_input = sum_n H_pre[n] H[n]; H_residual[n] = sum_m H_res[n,m] H[m]
    (reference src/mhc/_kernels.py:617-652).  Outputs take H's dtype."""
    if H.dim() != 4 or H.shape[2] != 4:
        raise ShapeError(f"H must be (batch, seq, 4, dim), got {tuple(H.shape)}")
    B, S, _, D = H.shape
    if tuple(H_pre.shape) != (B, 4) or tuple(H_res.shape) != (B, 4, 4):
        raise ShapeError(f"H_pre must be ({B}, 4) and H_res ({B}, 4, 4); got "
                         f"{tuple(H_pre.shape)}, {tuple(H_res.shape)}")
    dev = _lib.require_gpu(H, H_pre, H_res)
    H = H.contiguous()
    H_pre = _f32(H_pre)
    H_res = _f32(H_res)
    bi = torch.empty(B, S, D, device=dev, dtype=H.dtype)
    H_residual = torch.empty_like(H)
    lib = _lib.load()
    with _lib.on_device(dev):
        _lib.check(lib.mhc_stream_mix_forward(H.data_ptr(), H_pre.data_ptr(), H_res.data_ptr(), bi.data_ptr(),
                                              H_residual.data_ptr(), B, S, D, _lib.dtype_code(H),
                                              _lib.stream(dev)), "stream_mix_forward")
    return bi, H_residual


def add_residual_forward(H_residual: torch.Tensor, branch_output: torch.Tensor, H_post: torch.Tensor,
                         block_dim: int = 128) -> torch.Tensor:
    """H_new[n] = H_residual[n] + H_post[n] * branch_output (reference
    src/mhc/_kernels.py:655-687).  H_new takes H_residual's dtype."""
    if H_residual.dim() != 4 or H_residual.shape[2] != 4:
        raise ShapeError(f"H_residual must be (batch, seq, 4, dim), got {tuple(H_residual.shape)}")
    B, S, _, D = H_residual.shape
    if tuple(branch_output.shape) != (B, S, D) or tuple(H_post.shape) != (B, 4):
        raise ShapeError(f"branch_output must be ({B}, {S}, {D}) and H_post ({B}, 4); got "
                         f"{tuple(branch_output.shape)}, {tuple(H_post.shape)}")
    dev = _lib.require_gpu(H_residual, branch_output, H_post)
    H_residual = H_residual.contiguous()
    branch_output = branch_output.contiguous()
    H_post = _f32(H_post)
    H_new = torch.empty_like(H_residual)
    lib = _lib.load()
    with _lib.on_device(dev):
        _lib.check(lib.mhc_add_residual_forward(H_residual.data_ptr(), _lib.dtype_code(H_residual),
                                                branch_output.data_ptr(), _lib.dtype_code(branch_output),
                                                H_post.data_ptr(), H_new.data_ptr(), B, S, D, _lib.stream(dev)),
                   "add_residual_forward")
    return H_new


def fused_dynamic_weights_forward(
    x: torch.Tensor,
    phi: torch.Tensor,
    bias: torch.Tensor,
    alpha_pre: Union[float, torch.Tensor],
    alpha_post: Union[float, torch.Tensor],
    alpha_res: Union[float, torch.Tensor],
    sinkhorn_iters: int = 20,
    eps: float = 1e-6,
    return_aux: bool = False,
):
    """Eq. 14-19 in two kernels (reference src/mhc/_kernels.py:690-752).

    ``phi`` is read in its API layout [in_dim, 24] (no transposed copy) and the
    alphas may be device tensors (no host synchronisation).  Returns fp32
    ``(H_pre, H_post, H_res)``, plus ``aux`` [batch, 25] (raw projection and
    inv_rms, consumed by the backward) when ``return_aux``.
    """
    if x.dim() != 2:
        raise ShapeError(f"x must be (batch, in_dim), got {tuple(x.shape)}")
    R, K = x.shape
    if tuple(phi.shape) != (K, 24):
        raise ShapeError(f"phi shape mismatch: {tuple(phi.shape)} vs ({K}, 24)")
    if tuple(bias.shape) != (24,):
        raise ShapeError(f"bias shape mismatch: {tuple(bias.shape)} vs (24,)")
    if sinkhorn_iters < 0:
        raise ValueError("sinkhorn_iters must be >= 0")
    dev = _lib.require_gpu(x, phi, bias)
    x = x.contiguous()
    phi = _f32(phi)
    bias = _f32(bias)
    a = [_alpha_tensor(v, dev) for v in (alpha_pre, alpha_post, alpha_res)]
    H_pre = torch.empty(R, 4, device=dev, dtype=torch.float32)
    H_post = torch.empty(R, 4, device=dev, dtype=torch.float32)
    H_res = torch.empty(R, 4, 4, device=dev, dtype=torch.float32)
    aux = torch.empty(R, 25, device=dev, dtype=torch.float32)
    lib = _lib.load()
    ws = _lib.workspace(lib.mhc_dynamic_weights_workspace_bytes(R, K), dev)
    with _lib.on_device(dev):
        _lib.check(lib.mhc_dynamic_weights_forward(
            x.data_ptr(), _lib.dtype_code(x), phi.data_ptr(), bias.data_ptr(),
            a[0].data_ptr(), a[1].data_ptr(), a[2].data_ptr(),
            H_pre.data_ptr(), H_post.data_ptr(), H_res.data_ptr(), aux.data_ptr(),
            R, K, int(sinkhorn_iters), float(eps), _lib.ptr(ws), 0 if ws is None else ws.numel(),
            _lib.stream(dev)), "dynamic_weights_forward")
    if return_aux:
        return H_pre, H_post, H_res, aux
    return H_pre, H_post, H_res


def mean_pool(H: torch.Tensor) -> torch.Tensor:
    """x[b, n*D + d] = mean_s H[b, s, n, d] in fp32 (the reference's
    ``H.mean(dim=1).reshape(B, 4*D)``, src/mhc/module.py:123, without rounding
    x to H's dtype)."""
    if H.dim() != 4 or H.shape[2] != 4:
        raise ShapeError(f"H must be (batch, seq, 4, dim), got {tuple(H.shape)}")
    B, S, _, D = H.shape
    dev = _lib.require_gpu(H)
    H = H.contiguous()
    x = torch.empty(B, 4 * D, device=dev, dtype=torch.float32)
    lib = _lib.load()
    code = _lib.dtype_code(H)
    ws = _lib.workspace(lib.mhc_mean_pool_workspace_bytes(B, S, D, code), dev)
    with _lib.on_device(dev):
        _lib.check(lib.mhc_mean_pool(H.data_ptr(), code, x.data_ptr(), B, S, D, _lib.ptr(ws),
                                     0 if ws is None else ws.numel(), _lib.stream(dev)), "mean_pool")
    return x


def stream_expand(x: torch.Tensor, scale: float = 1.0, dtype: torch.dtype = None) -> torch.Tensor:
    """H[b,s,n,:] = scale * x[b,s,:] for the 4 streams, H in ``dtype`` (default x's).
    The backward of ``stream_collapse``.  No reference launcher: the reference
    takes the (batch, seq, 4, dim) state as given (README.md:38-39)."""
    if x.dim() != 3:
        raise ShapeError(f"x must be (batch, seq, dim), got {tuple(x.shape)}")
    B, S, D = x.shape
    dev = _lib.require_gpu(x)
    x = x.contiguous()
    H = torch.empty(B, S, 4, D, device=dev, dtype=dtype or x.dtype)
    lib = _lib.load()
    with _lib.on_device(dev):
        _lib.check(lib.mhc_stream_expand(x.data_ptr(), _lib.dtype_code(x), H.data_ptr(), _lib.dtype_code(H),
                                         B, S, D, float(scale), _lib.stream(dev)), "stream_expand")
    return H


def stream_collapse(H: torch.Tensor, scale: float = 1.0, dtype: torch.dtype = None) -> torch.Tensor:
    """y[b,s,:] = scale * sum_n H[b,s,n,:], y in ``dtype`` (default H's); scale 1/4
    is the stream mean.  The backward of ``stream_expand``."""
    if H.dim() != 4 or H.shape[2] != 4:
        raise ShapeError(f"H must be (batch, seq, 4, dim), got {tuple(H.shape)}")
    B, S, _, D = H.shape
    dev = _lib.require_gpu(H)
    H = H.contiguous()
    y = torch.empty(B, S, D, device=dev, dtype=dtype or H.dtype)
    lib = _lib.load()
    with _lib.on_device(dev):
        _lib.check(lib.mhc_stream_collapse(H.data_ptr(), _lib.dtype_code(H), y.data_ptr(), _lib.dtype_code(y),
                                           B, S, D, float(scale), _lib.stream(dev)), "stream_collapse")
    return y
