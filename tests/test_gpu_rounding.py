"""bf16 / fp16 outputs of the streaming kernels against the float64 value of the same
expression, rounded once (reference src/mhc/_kernels.py:137-310, _backward.py:269-496).

The oracle checks in test_gpu_ops.py / test_gpu_module.py hold these outputs to the
2e-2 normwise tolerance stated for bf16-input outputs.  That is the parity statement,
but it is about ten times one bf16 rounding (2^-9), so it cannot see truncation in place
of round-to-nearest-even or a weight rounded to the half format before use.  Here each
bulk output is compared with its defining expression evaluated in float64 from the
kernel's own inputs and fp32 weights (the weights the layer kernels computed, read back
through the launchers), then rounded once to the output dtype: every element must lie
within one unit in the last place plus the fp32 evaluation bound, and only a small
fraction may differ in bits (helpers.rounded_once_stats).
"""

import numpy as np
import pytest
import torch

from helpers import assert_rounded_once, rel_err, to_np
from oracle import mhc_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
HALF = [torch.bfloat16, torch.float16]


def _randn(g, shape, dtype=torch.float32, scale=1.0):
    return (torch.randn(shape, generator=g, device=DEV) * scale).to(dtype)


def _wsum(w, T):
    """sum_k w[b, k] T[b, :, k, :] for w [B, 4], written as broadcast products (no batched matmul)."""
    return sum(w[:, k, None, None] * T[:, :, k] for k in range(4))


def _mix_ref(H64, wpre, wres):
    """bi = sum_n pre[n] H[n], hr[n] = sum_m res[n, m] H[m], and their absolute-term sums."""
    A = H64.abs()
    bi, bia = _wsum(wpre, H64), _wsum(wpre.abs(), A)
    hr = torch.stack([_wsum(wres[:, n], H64) for n in range(4)], dim=2)
    hra = torch.stack([_wsum(wres[:, n].abs(), A) for n in range(4)], dim=2)
    return bi, bia, hr, hra


def _dh_ref(dbi64, dhn64, wpre, wres):
    """dH[m] = pre[m] d_bi + sum_n res[n, m] dH_new[n], and its absolute-term sum."""
    dH = torch.stack([wpre[:, m, None, None] * dbi64 + _wsum(wres[:, :, m], dhn64) for m in range(4)], dim=2)
    dHa = torch.stack([wpre[:, m, None, None].abs() * dbi64.abs() + _wsum(wres[:, :, m].abs(), dhn64.abs())
                       for m in range(4)], dim=2)
    return dH, dHa


def _red(a, T):
    """[B, 4]: sum over (s, d) of a[b, s, d] T[b, s, k, d]."""
    return torch.stack([(a * T[:, :, k]).sum(dim=(1, 2)) for k in range(4)], dim=1)


def _red44(A, T):
    """[B, 4, 4]: sum over (s, d) of A[b, s, n, d] T[b, s, m, d]."""
    return torch.stack([_red(A[:, :, n], T) for n in range(4)], dim=1)


@pytest.mark.parametrize("dtype", HALF)
@pytest.mark.parametrize("D", [512, 100])
def test_fused_stream_mix_rounds_once(dtype, D):
    import mhc

    g = torch.Generator(device=DEV)
    g.manual_seed(0)
    B, S = 3, 64
    H = _randn(g, (B, S, 4, D), dtype)
    H_pre = torch.rand((B, 4), generator=g, device=DEV)
    H_res = torch.rand((B, 4, 4), generator=g, device=DEV) - 0.3
    dbi = _randn(g, (B, S, D), dtype)
    dhr = _randn(g, (B, S, 4, D), dtype)
    Hl = H.clone().requires_grad_(True)
    pl, rl = H_pre.clone().requires_grad_(True), H_res.clone().requires_grad_(True)
    bi, hr = mhc.fused_stream_mix(Hl, pl, rl)
    torch.autograd.backward([bi, hr], [dbi, dhr])
    wpre, wres = H_pre.double(), H_res.double()
    bi64, bia, hr64, hra = _mix_ref(H.double(), wpre, wres)
    assert_rounded_once(bi, bi64, bia, "stream_mix bi")
    assert_rounded_once(hr, hr64, hra, "stream_mix H_residual")
    dH64, dHa = _dh_ref(dbi.double(), dhr.double(), wpre, wres)
    assert_rounded_once(Hl.grad, dH64, dHa, "stream_mix dH")
    dpre = _red(dbi.double(), H.double())
    dres = _red44(dhr.double(), H.double())
    assert rel_err(to_np(pl.grad), to_np(dpre)) < 1e-5 and rel_err(to_np(rl.grad), to_np(dres)) < 1e-5


@pytest.mark.parametrize("dtype", HALF)
@pytest.mark.parametrize("bo_dtype", ["same", torch.float32])
def test_fused_add_residual_rounds_once(dtype, bo_dtype):
    import mhc

    g = torch.Generator(device=DEV)
    g.manual_seed(1)
    B, S, D = 2, 48, 384
    bdt = dtype if bo_dtype == "same" else bo_dtype
    hr = _randn(g, (B, S, 4, D), dtype)
    bo = _randn(g, (B, S, D), bdt)
    H_post = 2 * torch.rand((B, 4), generator=g, device=DEV)
    dHn = _randn(g, (B, S, 4, D), dtype)
    bol, ql = bo.clone().requires_grad_(True), H_post.clone().requires_grad_(True)
    Hn = mhc.fused_add_residual(hr, bol, ql)
    Hn.backward(dHn)
    q = H_post.double()
    ref = hr.double() + q[:, None, :, None] * bo.double()[:, :, None, :]
    refa = hr.double().abs() + q.abs()[:, None, :, None] * bo.double().abs()[:, :, None, :]
    assert_rounded_once(Hn, ref, refa, "add_residual H_new")
    dbo = _wsum(q, dHn.double())
    dboa = _wsum(q.abs(), dHn.double().abs())
    if bdt == torch.float32:
        assert rel_err(to_np(bol.grad), to_np(dbo)) < 1e-6
    else:
        assert_rounded_once(bol.grad, dbo, dboa, "add_residual d_bo")
    dpost = _red(bo.double(), dHn.double())
    assert rel_err(to_np(ql.grad), to_np(dpost)) < 1e-5


def _layer_case(kind, dtype, B, S, D, seed):
    import mhc

    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    hc = mhc.HyperConnection(D, dynamic=kind != "static", use_fused_weights=kind == "dynamic").to(DEV)
    with torch.no_grad():
        if kind == "dynamic":
            hc.phi.copy_(_randn(g, (24, 4 * D), scale=0.02).T)
        elif kind == "unfused":
            for lin in (hc.W_pre, hc.W_post, hc.W_res):
                lin.weight.copy_(_randn(g, lin.weight.shape, scale=0.05))
        hc.H_res_base.copy_(_randn(g, (4, 4)))
    H = _randn(g, (B, S, 4, D), dtype)
    bo = _randn(g, (B, S, D), dtype)
    dHn = _randn(g, (B, S, 4, D), dtype)
    dbi = _randn(g, (B, S, D), dtype)
    return hc, H, bo, dHn, dbi


# The kernels' grad_x (the mean-pool's gradient, added to dH as grad_x / S) comes from fp32
# reductions over all S * D tokens, like the parameter gradients, and is held to the same
# fp32-gradient tolerance: an absolute allowance of GX_TOL times the largest |grad_x / S| of the
# float64 reference, on top of the rounding allowance of the rest of dH.
GX_TOL = 1e-4


def _unfused_weights_backward(hc, x, gw):
    """grad_x of the unfused weights (torch ops in fp32, as the layer runs them) for the packed
    weight gradient gw [B, 24]."""
    xl = x.detach().clone().requires_grad_(True)
    w = hc._unfused_weights_from(xl)
    (gx,) = torch.autograd.grad(w, xl, gw)
    return gx


def check_layer_rounding(kind, hc, H, bo, dHn, dbi):
    """Runs the layer's launchers (the ones HyperConnection.forward / backward call) and
    checks branch_input, H_new, d branch_output and dH against the once-rounded float64
    expressions built from the layer's own weights w [B, 24].  dH includes grad_x / S for
    the dynamic and unfused layers."""
    from mhc import _kernels, _layer

    B, S, _, D = H.shape
    if kind == "dynamic":
        params = (hc.phi, hc.H_pre_base, hc.H_post_base, hc.H_res_base, hc.alpha_pre, hc.alpha_post, hc.alpha_res)
        bi, x, w, aux = _layer.dynamic_forward(H, *params, hc.sinkhorn_iters, hc.eps)
    elif kind == "static":
        params = (hc.H_pre_base, hc.H_post_base, hc.H_res_base)
        bi, w = _layer.static_forward(H, *params, hc.sinkhorn_iters)
    else:
        x = _kernels.mean_pool(H)
        w = hc._unfused_weights_from(x).detach().float().contiguous()
        bi = _layer.branch_input(H, w)
    H_new = _layer.add_forward(H, bo, w)
    d_bo, dH_post = _layer.add_backward(dHn, bo, w)
    if kind == "dynamic":
        dH, *_ = _layer.dynamic_backward(H, dbi, dHn, dH_post, *params, x, w, aux, hc.sinkhorn_iters, hc.eps)
    elif kind == "static":
        dH, _ = _layer.static_backward(H, dbi, dHn, dH_post, *params, w, hc.sinkhorn_iters)
    else:
        _, dpre_k, dres_k = _layer.mix_backward(H, dbi, dHn, w, need_dH=False)
        gx_k = _unfused_weights_backward(hc, x, torch.cat([dpre_k, dH_post, dres_k], dim=1))
        dH = _layer.mix_dh(dbi, dHn, w, gx_k, H.shape, H.dtype)
    torch.cuda.synchronize()

    w64 = w.double()
    wpre, wpost, wres = w64[:, 0:4], w64[:, 4:8], w64[:, 8:24].reshape(B, 4, 4)
    H64, bo64, dHn64, dbi64 = H.double(), bo.double(), dHn.double(), dbi.double()
    bi64, bia, hr64, hra = _mix_ref(H64, wpre, wres)
    assert_rounded_once(bi, bi64, bia, f"{kind} layer bi")
    del bi64, bia
    hn = hr64 + wpost[:, None, :, None] * bo64[:, :, None, :]
    hna = hra + wpost.abs()[:, None, :, None] * bo64.abs()[:, :, None, :]
    del hr64, hra
    assert_rounded_once(H_new, hn, hna, f"{kind} layer H_new")
    del hn, hna
    dbo = _wsum(wpost, dHn64)
    dboa = _wsum(wpost.abs(), dHn64.abs())
    assert_rounded_once(d_bo, dbo, dboa, f"{kind} layer d_bo")
    del dbo, dboa
    dpost = _red(bo64, dHn64)
    assert rel_err(to_np(dH_post), to_np(dpost)) < 1e-5
    dH64, dHa = _dh_ref(dbi64, dHn64, wpre, wres)
    if kind != "static":
        # + grad_x / S, the mean-pool's share, with grad_x from the float64 weight backward fed
        # float64 reductions over all S * D tokens.
        dpre = _red(dbi64, H64)
        dres = _red44(dHn64, H64)
        if kind == "dynamic":
            bias = np.concatenate([to_np(hc.H_pre_base), to_np(hc.H_post_base), to_np(hc.H_res_base).reshape(16)])
            al = [float(to_np(a)[0]) for a in (hc.alpha_pre, hc.alpha_post, hc.alpha_res)]
            gx, *_ = O.dynamic_weights_backward(to_np(x), to_np(hc.phi), bias, *al, to_np(dpre), to_np(dH_post),
                                                to_np(dres), hc.sinkhorn_iters, hc.eps)
        else:
            p = {n.replace(".weight", ""): to_np(v) for n, v in hc.named_parameters()}
            gx = O.unfused_weights_backward(
                to_np(x), p["W_pre"], p["W_post"], p["W_res"], p["scale_pre"], p["scale_post"], p["scale_res"],
                p["H_pre_base"], p["H_post_base"], p["H_res_base"], to_np(dH_post), to_np(dpre), to_np(dres),
                hc.sinkhorn_iters, hc.eps)["x"]
        gxs = torch.tensor(gx, device=DEV).reshape(B, 1, 4, D) / S
        dH64 = dH64 + gxs
        # an absolute allowance of GX_TOL * max|grad_x / S|, expressed in the helper's terms
        # (it allows 8 * 2^-24 times the absolute-term sum)
        dHa = dHa + gxs.abs() + GX_TOL * float(gxs.abs().max()) * 2.0 ** 24 / 8
    assert_rounded_once(dH, dH64, dHa, f"{kind} layer dH")


@pytest.mark.parametrize("dtype", HALF)
@pytest.mark.parametrize("kind", ["dynamic", "static", "unfused"])
def test_layer_rounds_once(kind, dtype):
    hc, H, bo, dHn, dbi = _layer_case(kind, dtype, 2, 256, 448, seed=3)
    check_layer_rounding(kind, hc, H, bo, dHn, dbi)


@pytest.mark.parametrize("B,S,D,dtype", [(2048, 4, 1024, torch.bfloat16), (2048, 7, 1024, torch.float16),
                                         (2700, 5, 99, torch.bfloat16)])
def test_dh_many_short_sequences_rounds_once(B, S, D, dtype):
    """Pass C (mhc_layer_mix_dh) where a lane takes 4 tokens (S = 4) or 8 (S = 5 and 7; D = 99 on
    the scalar path), with grids of 1024 workgroups and more, against the float64 expression
    rounded once: dH[m] = pre[m] d_bi + sum_n res[n, m] dH_new[n] + grad_x[m] / S."""
    from mhc import _layer

    g = torch.Generator(device=DEV).manual_seed(11)
    dbi = _randn(g, (B, S, D), dtype)
    dHn = _randn(g, (B, S, 4, D), dtype)
    w = torch.rand((B, 24), generator=g, device=DEV)
    gx = _randn(g, (B, 4 * D))
    dH = _layer.mix_dh(dbi, dHn, w, gx, (B, S, 4, D), dtype)
    w64 = w.double()
    dH64, dHa = _dh_ref(dbi.double(), dHn.double(), w64[:, 0:4], w64[:, 8:24].reshape(B, 4, 4))
    gxs = gx.double().reshape(B, 1, 4, D) / S
    assert_rounded_once(dH, dH64 + gxs, dHa + gxs.abs(), f"dH B={B} S={S} D={D}")


def test_layer_rounds_once_ragged_dim():
    """D = 100: the scalar (one element per lane) path of every streaming kernel."""
    hc, H, bo, dHn, dbi = _layer_case("dynamic", torch.bfloat16, 3, 40, 100, seed=4)
    check_layer_rounding("dynamic", hc, H, bo, dHn, dbi)


@pytest.mark.parametrize("kind", ["dynamic", "unfused"])
def test_module_uses_the_checked_launchers(kind):
    """HyperConnection.forward / backward give the same bits as the launcher sequence that
    check_layer_rounding runs, so its checks hold for the module's full dH (grad_x / S
    included)."""
    from mhc import _kernels, _layer

    hc, H, bo, dHn, dbi = _layer_case(kind, torch.bfloat16, 2, 64, 256, seed=5)
    Hl, bol = H.clone().requires_grad_(True), bo.clone().requires_grad_(True)
    bi, add = hc(Hl)
    Hn = add(bol)
    torch.autograd.backward([Hn, bi], [dHn, dbi])
    if kind == "dynamic":
        params = (hc.phi, hc.H_pre_base, hc.H_post_base, hc.H_res_base, hc.alpha_pre, hc.alpha_post,
                  hc.alpha_res)
        bi2, x, w, aux = _layer.dynamic_forward(H, *params, hc.sinkhorn_iters, hc.eps)
        Hn2 = _layer.add_forward(H, bo, w)
        d_bo2, dpost = _layer.add_backward(dHn, bo, w)
        dH2, *_ = _layer.dynamic_backward(H, dbi, dHn, dpost, *params, x, w, aux, hc.sinkhorn_iters, hc.eps)
    else:
        x = _kernels.mean_pool(H)
        w = hc._unfused_weights_from(x).detach().float().contiguous()
        bi2 = _layer.branch_input(H, w)
        Hn2 = _layer.add_forward(H, bo, w)
        d_bo2, dpost = _layer.add_backward(dHn, bo, w)
        _, dpre, dres = _layer.mix_backward(H, dbi, dHn, w, need_dH=False)
        gx = _unfused_weights_backward(hc, x, torch.cat([dpre, dpost, dres], dim=1))
        dH2 = _layer.mix_dh(dbi, dHn, w, gx, H.shape, H.dtype)
    for a, b in ((bi, bi2), (Hn, Hn2), (bol.grad, d_bo2), (Hl.grad, dH2)):
        assert torch.equal(a, b)
