"""torch.library registrations, checked without a GPU.

Every ``torch.ops.mhc`` op runs here on fake CUDA tensors (shapes and dtypes
only, no kernel), and the traced layer's forward and backward run end to end in
fake mode: each gradient must come back with its input's shape and dtype.
The real kernels behind the same ops, torch.compile and ``opcheck`` are
exercised in tests/test_gpu_compile.py.
"""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import mhc
from mhc import _library

OPS = {
    "sinkhorn_forward", "sinkhorn_backward", "stream_mix_forward", "stream_mix_backward",
    "add_residual_forward", "add_residual_backward", "dynamic_weights_forward", "dynamic_weights_backward",
    "mean_pool", "layer_dynamic_forward", "layer_dynamic_backward", "layer_static_forward",
    "layer_static_backward", "layer_branch_input", "layer_mix_backward", "layer_add_forward",
    "layer_add_backward", "layer_mix_dh", "layer_mix_reduce", "stream_expand", "stream_collapse",
}
BF = torch.bfloat16
F32 = torch.float32


def sig(ts):
    return [(tuple(t.shape), t.dtype, t.device.type) for t in ts]


def test_every_launcher_is_registered():
    names = {n for n in dir(torch.ops.mhc) if not n.startswith("_") and n != "name"}
    assert names == OPS
    for n in OPS:
        assert torch._C._dispatch_has_kernel_for_dispatch_key(f"mhc::{n}", "CUDA"), n
        assert not torch._C._dispatch_has_kernel_for_dispatch_key(f"mhc::{n}", "CPU"), n


def test_fake_kernels_give_the_launchers_output_shapes_and_dtypes():
    B, S, D, R, K = 2, 8, 16, 3, 64
    with FakeTensorMode():
        e = lambda *s, dt=F32: torch.empty(*s, device="cuda", dtype=dt)  # noqa: E731
        H, bi, bo = e(B, S, 4, D, dt=BF), e(B, S, D, dt=BF), e(B, S, D, dt=torch.float16)
        pre, post, res = e(B, 4), e(B, 4), e(B, 4, 4)
        a = [e(1), e(1), e(1)]
        ops = torch.ops.mhc
        assert sig([ops.sinkhorn_forward(e(7, 4, 4, dt=BF), 20, 1e-8)]) == [((7, 4, 4), BF, "cuda")]
        assert sig([ops.sinkhorn_backward(e(7, 4, 4), e(7, 4, 4), 20, 1e-8)]) == [((7, 4, 4), F32, "cuda")]
        assert sig(ops.stream_mix_forward(H, pre, res)) == [((B, S, D), BF, "cuda"), ((B, S, 4, D), BF, "cuda")]
        assert sig(ops.stream_mix_backward(bi, H, H, pre, res)) == [
            ((B, S, 4, D), BF, "cuda"), ((B, 4), F32, "cuda"), ((B, 4, 4), F32, "cuda")]
        assert sig([ops.add_residual_forward(H, bo, post)]) == [((B, S, 4, D), BF, "cuda")]
        assert sig(ops.add_residual_backward(H, bo, post)) == [((B, S, D), torch.float16, "cuda"),
                                                               ((B, 4), F32, "cuda")]
        x = e(R, K, dt=BF)
        out = ops.dynamic_weights_forward(x, e(K, 24), e(24), *a, 20, 1e-6)
        assert sig(out) == [((R, 4), F32, "cuda"), ((R, 4), F32, "cuda"), ((R, 4, 4), F32, "cuda"),
                            ((R, 25), F32, "cuda")]
        g = ops.dynamic_weights_backward(x, e(K, 24), e(24), *a, e(R, 25), e(R, 4), e(R, 4), None, e(R, 4, 4),
                                         20, 1e-6)
        assert sig(g) == [((R, K), BF, "cuda"), ((K, 24), F32, "cuda"), ((24,), F32, "cuda"), ((3,), F32, "cuda")]
        assert sig([ops.mean_pool(H)]) == [((B, 4 * D), F32, "cuda")]
        base = [e(4), e(4), e(4, 4)]
        assert sig(ops.layer_dynamic_forward(H, e(4 * D, 24), *base, *a, 20, 1e-6)) == [
            ((B, S, D), BF, "cuda"), ((B, 4 * D), F32, "cuda"), ((B, 24), F32, "cuda"), ((B, 25), F32, "cuda")]
        assert sig(ops.layer_dynamic_backward(H, bi, None, None, e(4 * D, 24), *base, *a, e(B, 4 * D), e(B, 24),
                                              e(B, 25), 20, 1e-6)) == [
            ((B, S, 4, D), BF, "cuda"), ((4 * D, 24), F32, "cuda"), ((24,), F32, "cuda"), ((3,), F32, "cuda")]
        assert sig(ops.layer_static_forward(H, *base, 20)) == [((B, S, D), BF, "cuda"), ((B, 24), F32, "cuda")]
        assert sig(ops.layer_static_backward(H, bi, H, e(B, 4), *base, e(B, 24), 20)) == [
            ((B, S, 4, D), BF, "cuda"), ((24,), F32, "cuda")]
        assert sig([ops.layer_branch_input(H, e(B, 24))]) == [((B, S, D), BF, "cuda")]
        assert sig(ops.layer_mix_backward(H, bi, H, e(B, 24))) == [
            ((B, S, 4, D), BF, "cuda"), ((B, 4), F32, "cuda"), ((B, 16), F32, "cuda")]
        assert sig(ops.layer_mix_reduce(H, bi, H, e(B, 24))) == [((B, 4), F32, "cuda"), ((B, 16), F32, "cuda")]
        assert sig(ops.layer_mix_reduce(H, None, None, e(B, 24))) == [((B, 4), F32, "cuda"), ((B, 16), F32, "cuda")]
        assert sig([ops.layer_mix_dh(bi, H, e(B, 24), e(B, 4 * D), H)]) == [((B, S, 4, D), BF, "cuda")]
        assert sig([ops.layer_mix_dh(None, None, e(B, 24), None, H)]) == [((B, S, 4, D), BF, "cuda")]
        assert sig([ops.layer_add_forward(H, bo, e(B, 24))]) == [((B, S, 4, D), BF, "cuda")]
        assert sig(ops.layer_add_backward(H, bo, e(B, 24))) == [((B, S, D), torch.float16, "cuda"),
                                                                ((B, 4), F32, "cuda")]
        assert sig([ops.stream_expand(bo, 1.0)]) == [((B, S, 4, D), torch.float16, "cuda")]
        assert sig([ops.stream_expand(bo, 1.0, BF)]) == [((B, S, 4, D), BF, "cuda")]
        assert sig([ops.stream_collapse(H, 0.25)]) == [((B, S, D), BF, "cuda")]
        assert sig([ops.stream_collapse(H, 0.25, F32)]) == [((B, S, D), F32, "cuda")]


@pytest.mark.parametrize("dynamic,fused", [(True, True), (False, True), (True, False)])
@pytest.mark.parametrize("calls", [0, 1, 2])
def test_traced_layer_wiring_in_fake_mode(dynamic, fused, calls):
    """The traced layer (link output instead of the side channel) returns one gradient
    per input, each shaped and typed like it, however often the closure is called.
    Meta tensors run the ops' fake kernels and, unlike fake CUDA tensors, let the
    autograd engine run without a device."""
    B, S, D = 2, 8, 16
    hc = mhc.HyperConnection(D, dynamic=dynamic, use_fused_weights=fused).to("meta")
    H = torch.empty(B, S, 4, D, device="meta", dtype=BF, requires_grad=True)
    bi, add = hc._forward_traced(H)
    outs, grads = [bi], [torch.empty_like(bi)]
    for _ in range(calls):
        bo = torch.empty(B, S, D, device="meta", dtype=BF, requires_grad=True)
        Hn = add(bo)
        assert sig([Hn]) == [((B, S, 4, D), BF, "meta")]
        outs.append(Hn)
        grads.append(torch.empty_like(Hn))
    params = [p for p in hc.parameters()]
    gs = torch.autograd.grad(outs, [H, *params], grads, allow_unused=True)
    assert sig([gs[0]]) == [((B, S, 4, D), BF, "meta")]
    for p, g in zip(params, gs[1:]):
        assert g is not None and g.shape == p.shape and g.dtype == p.dtype


def test_public_ops_trace_to_registered_ops():
    """Under torch.compile the public ops route to torch.ops.mhc.* with autograd."""
    import inspect

    from mhc import module, ops

    for fn in (ops.sinkhorn_knopp, ops.fused_stream_mix, ops.fused_add_residual, ops.fused_dynamic_weights):
        src = inspect.getsource(fn)
        assert "torch.compiler.is_compiling()" in src and "torch.ops.mhc." in src, fn.__name__
    assert "self._forward_traced(H)" in inspect.getsource(module.HyperConnection.forward)
    for op in ("sinkhorn_forward", "stream_mix_forward", "add_residual_forward", "dynamic_weights_forward",
               "mean_pool", "stream_expand", "stream_collapse"):
        assert torch._C._dispatch_has_kernel_for_dispatch_key(f"mhc::{op}", "Autograd"), op
    assert _library.LayerAdd is not None
