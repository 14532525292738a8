"""GPU parity of the stream expand / collapse ops (mhc.streams, mhc_stream_expand /
mhc_stream_collapse) against the float64 oracle and against torch fp32 expressions
evaluated in the kernels' order (expand: one fp32 product, one rounding; collapse:
((h0 + h1) + h2) + h3 in fp32, times scale, one rounding), which must match bit for
bit.  Gradients go through autograd: each op's backward is the other op.
"""

import numpy as np
import pytest
import torch

from helpers import rel_err, to_np
from oracle import mhc_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _expand_ref(x, scale, dtype):
    return (x.float() * scale).to(dtype).unsqueeze(2).expand(-1, -1, 4, -1).contiguous()


def _collapse_ref(H, scale, dtype):
    h = H.float()
    return ((((h[:, :, 0] + h[:, :, 1]) + h[:, :, 2]) + h[:, :, 3]) * scale).to(dtype)


@pytest.mark.parametrize("D", [256, 100, 37])
@pytest.mark.parametrize("dt_in", DTYPES)
@pytest.mark.parametrize("dt_out", DTYPES)
def test_expand_and_collapse_bitwise_and_oracle(D, dt_in, dt_out):
    from mhc import _kernels as K

    g = torch.Generator().manual_seed(D)
    B, S = 3, 41
    x = torch.randn((B, S, D), generator=g).to(dt_in).to(DEV)
    H = torch.randn((B, S, 4, D), generator=g).to(dt_in).to(DEV)
    for scale in (1.0, 0.25, -1.5):
        He = K.stream_expand(x, scale, dt_out)
        assert He.dtype == dt_out and He.shape == (B, S, 4, D)
        assert torch.equal(He, _expand_ref(x, scale, dt_out))
        tol = 1e-6 if dt_out == torch.float32 else 1e-2
        assert rel_err(to_np(He), O.stream_expand(to_np(x), scale)) < tol
        y = K.stream_collapse(H, scale, dt_out)
        assert y.dtype == dt_out and y.shape == (B, S, D)
        assert torch.equal(y, _collapse_ref(H, scale, dt_out))
        assert rel_err(to_np(y), O.stream_collapse(to_np(H), scale)) < tol


@pytest.mark.parametrize("dtype", DTYPES)
def test_expand_collapse_autograd_against_oracle(dtype):
    import mhc

    g = torch.Generator().manual_seed(7)
    B, S, D = 2, 33, 264
    x = torch.randn((B, S, D), generator=g).to(dtype).to(DEV).requires_grad_(True)
    gy = torch.randn((B, S, D), generator=g).to(dtype).to(DEV)
    H = mhc.streams.expand_streams(x)
    Hs = H * torch.arange(1, 5, device=DEV, dtype=dtype).view(1, 1, 4, 1)  # make the streams differ
    y = mhc.streams.collapse_streams(Hs, reduction="mean")
    y.backward(gy)
    # y = mean_n (n+1) x = 2.5 x, dx = 2.5 gy
    tol = 1e-6 if dtype == torch.float32 else 1e-2
    assert rel_err(to_np(y), 2.5 * to_np(x)) < tol
    dHs = O.stream_collapse_backward(to_np(gy), 0.25)
    dx = O.stream_expand_backward(dHs * np.arange(1, 5).reshape(1, 1, 4, 1), 1.0)
    assert x.grad.dtype == dtype
    assert rel_err(to_np(x.grad), dx) < tol
    ys = mhc.streams.collapse_streams(H.detach().requires_grad_(True), reduction="sum")
    assert torch.equal(ys, _collapse_ref(H.detach(), 1.0, dtype))


def test_mixed_dtype_gradients_come_back_in_the_input_dtype():
    import mhc

    x = torch.randn(2, 8, 64, device=DEV, dtype=torch.float32, requires_grad=True)
    H = mhc.streams.expand_streams(x, dtype=torch.bfloat16)
    assert H.dtype == torch.bfloat16
    y = mhc.streams.collapse_streams(H, dtype=torch.float32)
    assert y.dtype == torch.float32
    y.sum().backward()
    assert x.grad.dtype == torch.float32
    assert torch.equal(x.grad, torch.ones_like(x))  # mean of 4 copies: d/dx = 1


def test_empty_and_bad_arguments():
    import mhc
    from mhc import _kernels as K

    for shape in [(0, 4, 8), (2, 0, 8), (2, 4, 0)]:
        x = torch.empty(shape, device=DEV, dtype=torch.bfloat16)
        assert K.stream_expand(x).shape == (shape[0], shape[1], 4, shape[2])
        assert K.stream_collapse(K.stream_expand(x)).shape == shape
    with pytest.raises(AssertionError):
        K.stream_collapse(torch.zeros(2, 3, 5, 8, device=DEV))
    with pytest.raises(ValueError):
        mhc.streams.collapse_streams(torch.zeros(2, 3, 4, 8, device=DEV), reduction="max")
    with pytest.raises(ValueError):
        mhc.streams.expand_streams(torch.zeros(2, 3, 8, device=DEV), num_streams=2)
    with pytest.raises(RuntimeError):
        K.stream_expand(torch.zeros(2, 3, 8))


def test_full_size_config3_round_trip():
    """At config-3 size (B=4, S=4096, D=4096 bf16): collapse(expand(x), mean) == x
    exactly (four equal bf16 values average to themselves), and the sum of the
    expanded tensor's streams is 4x (exact in fp32, one rounding)."""
    from mhc import _kernels as K

    g = torch.Generator(device=DEV).manual_seed(3)
    x = torch.randn((4, 4096, 4096), generator=g, device=DEV).bfloat16()
    H = K.stream_expand(x)
    assert torch.equal(K.stream_collapse(H, 0.25), x)
    assert torch.equal(K.stream_collapse(H, 1.0), (x.float() * 4).bfloat16())
    del H
