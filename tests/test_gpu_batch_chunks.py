"""Batches beyond the 65,535 that one launch's grid.y can hold.

The reference launches grid = (batch * seq, ...) in one go (reference
src/mhc/_kernels.py:643,678; _backward.py:562,612), so a caller may pass any batch.  The
streaming kernels here put the batch on grid.y and split larger batches into several
launches (for_batch_chunks), each with its first batch b0 entering every index and every
per-batch partial record.  B = 65,537 with a tiny S * D makes the second launch (b0 =
65,535, two batches) run in every such entry point: the mixing and add kernels, their
reductions, the mean-pool, pass C and the static pass BC, and expand / collapse.  Results
are checked against the float64 oracle over the whole batch and over the last two batches
alone, where a wrong b0 would land.
"""

import numpy as np
import pytest
import torch

from helpers import rel_err, to_np
from oracle import mhc_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
B = 65537
S = 2
CASES = [(torch.float32, 8), (torch.bfloat16, 8), (torch.float32, 5)]  # 16-byte vectors, and D = 5 scalar


def _tol(dtype):
    """(forward, bulk gradient, parameter / weight gradient) tolerances."""
    return (1e-5, 1e-4, 1e-4) if dtype == torch.float32 else (2e-2, 2e-2, 1e-4)


def _check(got, want, tol, what):
    got = to_np(got).reshape(np.shape(want))
    errs = (rel_err(got, want), rel_err(got[-2:], want[-2:]))
    print(f"B={B} {what}: {errs[0]:.2e} (last two batches {errs[1]:.2e})", flush=True)
    assert errs[0] < tol and errs[1] < tol, (what, errs)


def _inputs(dtype, D, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    mk = lambda *shape: torch.randn(shape, generator=g, device=DEV).to(dtype)  # noqa: E731
    return g, mk(B, S, 4, D), mk(B, S, D), mk(B, S, 4, D), mk(B, S, D)


@pytest.mark.parametrize("dtype,D", CASES)
def test_stream_ops_beyond_one_launch(dtype, D):
    import mhc

    ftol, gtol, wtol = _tol(dtype)
    g, H, bo, dHn, dbi = _inputs(dtype, D, 0)
    pre = torch.rand((B, 4), generator=g, device=DEV)
    res = torch.rand((B, 4, 4), generator=g, device=DEV)
    post = 2 * torch.rand((B, 4), generator=g, device=DEV)
    Hl, pl, rl = H.clone().requires_grad_(True), pre.clone().requires_grad_(True), res.clone().requires_grad_(True)
    bi, hr = mhc.fused_stream_mix(Hl, pl, rl)
    torch.autograd.backward([bi, hr], [dbi, dHn])
    obi, ohr = O.stream_mix(to_np(H), to_np(pre), to_np(res))
    odH, opre, ores = O.stream_mix_backward(to_np(dbi), to_np(dHn), to_np(H), to_np(pre), to_np(res))
    _check(bi, obi, ftol, "stream_mix bi")
    _check(hr, ohr, ftol, "stream_mix H_residual")
    _check(Hl.grad, odH, gtol, "stream_mix dH")
    _check(pl.grad, opre, wtol, "stream_mix dH_pre")
    _check(rl.grad, ores, wtol, "stream_mix dH_res")

    rl2, bol, ql = H.clone(), bo.clone().requires_grad_(True), post.clone().requires_grad_(True)
    Hn = mhc.fused_add_residual(rl2, bol, ql)
    Hn.backward(dHn)
    oHn = O.add_residual(to_np(H), to_np(bo), to_np(post))
    _, obo, opost = O.add_residual_backward(to_np(dHn), to_np(bo), to_np(post))
    _check(Hn, oHn, ftol, "add_residual H_new")
    _check(bol.grad, obo, gtol, "add_residual d_bo")
    _check(ql.grad, opost, wtol, "add_residual dH_post")

    x = bo.clone().requires_grad_(True)
    Hx = mhc.streams.expand_streams(x, scale=0.5)
    y = mhc.streams.collapse_streams(Hx, reduction="sum")
    y.backward(dbi)
    _check(Hx, O.stream_expand(to_np(bo), 0.5), ftol, "expand")
    _check(y, O.stream_collapse(O.stream_expand(to_np(bo), 0.5), 1.0), ftol, "collapse")
    _check(x.grad, O.stream_expand_backward(O.stream_collapse_backward(to_np(dbi), 1.0), 0.5), gtol,
           "expand / collapse backward")


@pytest.mark.parametrize("kind", ["dynamic", "static", "unfused"])
@pytest.mark.parametrize("dtype,D", CASES)
def test_layer_beyond_one_launch(kind, dtype, D):
    import mhc

    ftol, gtol, ptol = _tol(dtype)
    g, H, bo, dHn, dbi = _inputs(dtype, D, 1)
    hc = mhc.HyperConnection(D, dynamic=kind != "static", use_fused_weights=kind == "dynamic").to(DEV)
    with torch.no_grad():
        for p in hc.parameters():
            p.add_(torch.randn(p.shape, generator=g, device=DEV) * 0.05)
    Hl, bol = H.clone().requires_grad_(True), bo.clone().requires_grad_(True)
    bi, add = hc(Hl)
    Hn = add(bol)
    torch.autograd.backward([Hn, bi], [dHn, dbi])
    p = {n.replace(".weight", ""): to_np(v) for n, v in hc.named_parameters()}
    obi, oHn, cache = O.layer_forward(p, to_np(H), to_np(bo), kind != "static", kind != "unfused",
                                      hc.sinkhorn_iters, hc.eps)
    og = {k.replace(".weight", ""): v for k, v in O.layer_backward(p, cache, to_np(dHn), to_np(dbi)).items()}
    _check(bi, obi, ftol, f"{kind} layer bi")
    _check(Hn, oHn, ftol, f"{kind} layer H_new")
    _check(Hl.grad, og["H"], gtol, f"{kind} layer dH")
    _check(bol.grad, og["bo"], gtol, f"{kind} layer d_bo")
    for n, prm in hc.named_parameters():
        n = n.replace(".weight", "")
        err = rel_err(to_np(prm.grad).reshape(np.shape(og[n])), og[n])
        print(f"B={B} {kind} layer d{n}: {err:.2e}", flush=True)
        assert err < ptol, n
