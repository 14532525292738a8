"""GPU parity of mhc.HyperConnection (forward and every gradient) against the
float64 oracle layer, plus the closure / autograd edge cases.

Inputs follow one draw order from a CPU generator seeded with 0:
H, phi, H_res_base, branch_output, dH_new, d_branch_input.
"""

import numpy as np
import pytest
import torch

from helpers import rel_err, to_np
from oracle import mhc_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


def make_case(B, S, D, dtype, dynamic=True, fused=True, phi_std=None, res_std=None, seed=0, layer_idx=0):
    import mhc

    g = torch.Generator()
    g.manual_seed(seed)
    H = torch.randn((B, S, 4, D), generator=g).to(dtype)
    hc = mhc.HyperConnection(D, dynamic=dynamic, use_fused_weights=fused, layer_idx=layer_idx)
    if phi_std is not None and dynamic and fused:
        phi_t = torch.randn((24, 4 * D), generator=g) * phi_std  # [24, 4D], transposed to the API layout
        with torch.no_grad():
            hc.phi.copy_(phi_t.T)
    if phi_std is not None and dynamic and not fused:
        with torch.no_grad():
            for lin in (hc.W_pre, hc.W_post, hc.W_res):
                lin.weight.copy_(torch.randn(lin.weight.shape, generator=g) * phi_std)
    if res_std is not None:
        with torch.no_grad():
            hc.H_res_base.copy_(torch.randn((4, 4), generator=g) * res_std)
    bo = torch.randn((B, S, D), generator=g).to(dtype)
    dHn = torch.randn((B, S, 4, D), generator=g).to(dtype)
    dbi = torch.randn((B, S, D), generator=g).to(dtype)
    return hc.to(DEV), H.to(DEV), bo.to(DEV), dHn.to(DEV), dbi.to(DEV)


def params_np(hc):
    return {n.replace(".weight", ""): to_np(p) for n, p in hc.named_parameters()}


def run_gpu(hc, H, bo, dHn, dbi, copy=torch.clone):
    Hl = copy(H).requires_grad_(True)
    bol = copy(bo).requires_grad_(True)
    hc.zero_grad(set_to_none=True)
    bi, add = hc(Hl)
    Hn = add(bol)
    torch.autograd.backward([Hn, bi], [dHn, dbi])
    grads = {n.replace(".weight", ""): p.grad for n, p in hc.named_parameters()}
    grads["H"] = Hl.grad
    grads["bo"] = bol.grad
    return bi, Hn, grads


def check_layer(hc, H, bo, dHn, dbi, fwd_tol, h_tol, p_tol, copy=torch.clone):
    bi, Hn, grads = run_gpu(hc, H, bo, dHn, dbi, copy)
    p = params_np(hc)
    obi, oHn, cache = O.layer_forward(p, to_np(H), to_np(bo), hc.dynamic, hc.use_fused_weights or not hc.dynamic,
                                      hc.sinkhorn_iters, hc.eps)
    og = {k.replace(".weight", ""): v for k, v in O.layer_backward(p, cache, to_np(dHn), to_np(dbi)).items()}
    errs = {"bi": rel_err(to_np(bi), obi), "H_new": rel_err(to_np(Hn), oHn)}
    for k, v in og.items():
        errs["d" + k] = rel_err(to_np(grads[k]).reshape(np.shape(v)), v)
    print("layer errors:", {k: f"{e:.2e}" for k, e in errs.items()}, flush=True)
    assert bi.dtype == H.dtype and Hn.dtype == H.dtype
    assert errs["bi"] < fwd_tol and errs["H_new"] < fwd_tol, errs
    assert errs["dH"] < h_tol and errs["dbo"] < h_tol, errs
    for k, e in errs.items():
        if k not in ("bi", "H_new", "dH", "dbo"):
            assert e < p_tol, (k, errs)
    return errs


@pytest.mark.parametrize("phi_std", [None, 0.02])
def test_config1_fp32_dynamic(phi_std):
    """Config 1: dim 512, fp32, H (2, 128, 4, 512); default init (phi = 0, the
    sgn(0) case in the Sinkhorn backward) and phi ~ N(0, 0.02)."""
    hc, H, bo, dHn, dbi = make_case(2, 128, 512, torch.float32, phi_std=phi_std)
    check_layer(hc, H, bo, dHn, dbi, 1e-5, 1e-4, 1e-4)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_dynamic_low_precision(dtype):
    """Config 3 / 4 at reduced size: bf16 / fp16 H, fp32 parameters."""
    hc, H, bo, dHn, dbi = make_case(2, 96, 448, dtype, phi_std=0.02)
    check_layer(hc, H, bo, dHn, dbi, 2e-2, 2e-2, 1e-4)


def test_static_fp16():
    """Config 5 at reduced size: dynamic=False, fp16 H, H_res_base ~ N(0, 1)."""
    hc, H, bo, dHn, dbi = make_case(4, 64, 256, torch.float16, dynamic=False, res_std=1.0)
    check_layer(hc, H, bo, dHn, dbi, 2e-2, 2e-2, 1e-4)


def test_static_fp32():
    hc, H, bo, dHn, dbi = make_case(2, 33, 96, torch.float32, dynamic=False, res_std=1.0, layer_idx=2)
    check_layer(hc, H, bo, dHn, dbi, 1e-5, 1e-4, 1e-4)


def test_unfused_dynamic_fp32():
    hc, H, bo, dHn, dbi = make_case(2, 40, 64, torch.float32, fused=False, phi_std=0.05)
    check_layer(hc, H, bo, dHn, dbi, 1e-5, 1e-4, 1e-4)


@pytest.mark.parametrize("B,S,D,dtype", [(1, 1, 4096, torch.bfloat16), (3, 2, 100, torch.bfloat16),
                                         (64, 1, 256, torch.float32), (2, 8, 448, torch.float16),
                                         (4, 7, 96, torch.float32), (2, 9, 64, torch.bfloat16),
                                         (200, 3, 128, torch.bfloat16), (512, 1, 128, torch.float32),
                                         (600, 2, 64, torch.bfloat16), (515, 12, 32, torch.float16),
                                         (520, 1, 99, torch.bfloat16), (70, 2, 99, torch.float32),
                                         (96, 1, 256, torch.float16), (600, 1, 128, torch.bfloat16),
                                         (6, 5, 99, torch.bfloat16), (40, 16, 64, torch.float16),
                                         (80, 1, 128, torch.bfloat16), (300, 3, 64, torch.bfloat16),
                                         (512, 2, 1024, torch.bfloat16), (66, 3, 8192, torch.float16)])
def test_short_sequences(B, S, D, dtype):
    """Decode-like sequence lengths and batches of many sequences: S up to 8 takes the
    single-launch mean-pool (colsum_direct_kernel), S = 9 and 12 the two-kernel one; from 64
    batches the weights backward runs on the MFMA kernel in row chunks, and the projection too
    at S = 1 (on H's rows), for S > 1 once B * D reaches 2^19 (on the pooled rows); D = 99 (4D % 16 = 12) keeps the folded projection and the scalar
    mean-pool, with the backward's MFMA pass on ragged column blocks.  (Pass C's 4 and 8 tokens
    per lane at S = 3-16 need grids of 1024 workgroups: test_gpu_rounding covers them.)  Dynamic
    fused weights, phi ~ N(0, 0.02)."""
    hc, H, bo, dHn, dbi = make_case(B, S, D, dtype, phi_std=0.02)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    check_layer(hc, H, bo, dHn, dbi, tol, 1e-4 if dtype == torch.float32 else 2e-2, 1e-4)


@pytest.mark.parametrize("B,S,D,dtype", [(600, 1, 128, torch.bfloat16), (520, 3, 64, torch.bfloat16),
                                         (8, 4, 256, torch.float32), (3, 20, 96, torch.bfloat16),
                                         (512, 1, 64, torch.float16), (530, 1, 99, torch.bfloat16),
                                         (100, 1, 128, torch.bfloat16), (300, 4, 64, torch.bfloat16),
                                         (260, 4, 2048, torch.bfloat16)])
def test_no_grad_forward_matches_grad_forward(B, S, D, dtype):
    """A forward no gradient reaches keeps no pooled rows x (at S = 1 with many batches it never
    forms them: the projection reads H's rows); branch_input and the closure's H_new come out
    bit for bit as in a forward that keeps x for a backward."""
    hc, H, bo, _, _ = make_case(B, S, D, dtype, phi_std=0.02)
    bi, add = hc(H.clone().requires_grad_(True))
    Hn = add(bo)
    with torch.no_grad():
        bi0, add0 = hc(H)
        Hn0 = add0(bo)
    assert torch.equal(bi0, bi.detach()) and torch.equal(Hn0, Hn.detach())
    # and the no-grad forward against the oracle
    obi, oHn, _ = O.layer_forward(params_np(hc), to_np(H), to_np(bo), True, True, hc.sinkhorn_iters, hc.eps)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert rel_err(to_np(bi0), obi) < tol and rel_err(to_np(Hn0), oHn) < tol


@pytest.mark.parametrize("B,D,dtype", [(5, 256, torch.bfloat16), (96, 256, torch.float16),
                                       (600, 128, torch.bfloat16), (70, 99, torch.bfloat16),
                                       (80, 64, torch.float32)])
def test_s1_backward_reads_h_rows(B, D, dtype):
    """At S = 1 the training forward keeps no pooled rows: the backward reads H's rows in H's dtype
    (x = H exactly, as the mean of one row).  Its gradients against the same backward given x in
    f32: the same bits where both run the same pass (below 64 batches the one-chunk VALU pass,
    above it the MFMA pass, whose 16-bit x is one bf16 term where f32 x is hi + a zero mid); D = 99
    in bf16 (4D % 8 = 4) leaves the 16-bit rows to the VALU pass, to fp32 tolerance."""
    from mhc import _layer

    hc, H, _, dHn, dbi = make_case(B, 1, D, dtype, phi_std=0.02)
    params = [hc.phi, hc.H_pre_base, hc.H_post_base, hc.H_res_base, hc.alpha_pre, hc.alpha_post, hc.alpha_res]
    params = [p.detach() for p in params]
    bi, x, w, aux = _layer.dynamic_forward(H, *params, hc.sinkhorn_iters, hc.eps)
    bi0, x0, w0, aux0 = _layer.dynamic_forward(H, *params, hc.sinkhorn_iters, hc.eps, keep_x=False)
    assert x0 is None and torch.equal(x, H.float().reshape(B, 4 * D))
    assert torch.equal(bi, bi0) and torch.equal(w, w0) and torch.equal(aux, aux0)
    dpost = torch.randn((B, 4), device=DEV)
    got = _layer.dynamic_backward(H, dbi, dHn, dpost, *params, None, w, aux, hc.sinkhorn_iters, hc.eps)
    want = _layer.dynamic_backward(H, dbi, dHn, dpost, *params, x, w, aux, hc.sinkhorn_iters, hc.eps)
    exact = dtype == torch.float32 or D % 2 == 0
    for name, g, t in zip(("dH", "grad_phi", "grad_bias", "grad_alpha"), got, want):
        if exact:
            assert torch.equal(g, t), name
        else:
            # fp32 sums in another order; dH (bf16) then rounds a few elements the other way
            e = rel_err(to_np(g), to_np(t))
            print(f"{name}: {e:.2e}", flush=True)
            assert e < (1e-2 if name == "dH" else 1e-5), (name, e)
    with pytest.raises(ValueError):
        _layer.dynamic_backward(H.expand(B, 2, 4, D), dbi.expand(B, 2, D), None, None, *params, None, w, aux,
                                hc.sinkhorn_iters, hc.eps)


def test_ragged_dim_bf16():
    """D not a multiple of the 8-element vector: the scalar-path kernels."""
    hc, H, bo, dHn, dbi = make_case(3, 17, 100, torch.bfloat16, phi_std=0.02)
    check_layer(hc, H, bo, dHn, dbi, 2e-2, 2e-2, 1e-4)


@pytest.mark.parametrize("dynamic,fused", [(True, True), (False, True), (True, False)])
def test_compute_weights_matches_oracle_and_layer(dynamic, fused):
    """_compute_weights returns the oracle layer's (H_post, H_pre, H_res); the layer mixes
    with the same H_pre; gradients reach every parameter."""
    hc, H, bo, _, _ = make_case(2, 16, 64, torch.float32, dynamic=dynamic, fused=fused, phi_std=0.05,
                                res_std=0.5, layer_idx=1)
    H_post, H_pre, H_res = hc._compute_weights(H)
    _, _, cache = O.layer_forward(params_np(hc), to_np(H), to_np(bo), dynamic, fused or not dynamic,
                                  hc.sinkhorn_iters, hc.eps)
    assert H_post.shape == (2, 4) and H_pre.shape == (2, 4) and H_res.shape == (2, 4, 4)
    for got, key in ((H_post, "H_post"), (H_pre, "H_pre"), (H_res, "H_res")):
        assert got.dtype == torch.float32
        assert rel_err(to_np(got), np.broadcast_to(cache[key], got.shape)) < 1e-5, key
    bi, _ = hc(H)
    bi_ref = (H_pre.detach()[:, None, :, None] * H).sum(dim=2)
    assert rel_err(to_np(bi), to_np(bi_ref)) < 1e-5
    (H_post.sum() + H_pre.square().sum() + H_res.square().sum()).backward()
    for name, p in hc.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all(), name


def test_non_contiguous_inputs():
    """H as a transposed view and branch_output as a strided slice: the layer copies what it
    must and matches the oracle; gradients come back in the inputs' shapes."""
    hc, H, bo, dHn, dbi = make_case(2, 24, 64, torch.float32, phi_std=0.05)
    Ht = H.permute(0, 1, 3, 2).contiguous().permute(0, 1, 3, 2)  # same values, [B,S,4,D] view of [B,S,D,4]
    assert not Ht.is_contiguous()
    wide = torch.zeros(2, 24, 2 * 64, device=DEV)
    wide[:, :, ::2] = bo
    bos = wide[:, :, ::2]
    assert not bos.is_contiguous()
    Hl = Ht.detach().requires_grad_(True)
    bol = bos.detach().requires_grad_(True)
    bi, add = hc(Hl)
    Hn = add(bol)
    torch.autograd.backward([Hn, bi], [dHn, dbi])
    p = params_np(hc)
    obi, oHn, cache = O.layer_forward(p, to_np(H), to_np(bo))
    og = O.layer_backward(p, cache, to_np(dHn), to_np(dbi))
    assert rel_err(to_np(bi), obi) < 1e-5 and rel_err(to_np(Hn), oHn) < 1e-5
    assert Hl.grad.shape == Hl.shape and bol.grad.shape == bol.shape
    assert rel_err(to_np(Hl.grad), og["H"]) < 1e-4 and rel_err(to_np(bol.grad), og["bo"]) < 1e-4


@pytest.mark.parametrize("dynamic", [False, True])
def test_empty_sequence(dynamic):
    """S = 0: empty outputs and no launch errors.  dH_post is an empty sum, so the static layer's
    H_post_base gradient is exactly zero (the dynamic layer's mean over no tokens is NaN, as
    torch's H.mean is)."""
    import mhc

    hc = mhc.HyperConnection(64, dynamic=dynamic).to(DEV)
    H = torch.zeros((2, 0, 4, 64), device=DEV, requires_grad=True)
    bo = torch.zeros((2, 0, 64), device=DEV, requires_grad=True)
    bi, add = hc(H)
    Hn = add(bo)
    assert bi.shape == (2, 0, 64) and Hn.shape == (2, 0, 4, 64)
    (Hn.sum() + bi.sum()).backward()
    torch.cuda.synchronize()
    assert H.grad.shape == H.shape and bo.grad.shape == bo.shape
    if not dynamic:
        assert float(hc.H_post_base.grad.abs().sum()) == 0.0


@pytest.mark.parametrize("dynamic,fused", [(True, True), (False, True), (True, False)])
def test_empty_batch(dynamic, fused):
    """B = 0: empty outputs, and every parameter gradient an empty sum, exactly zero (as torch's
    sums over no rows are), not what the gradient buffers held before."""
    import mhc

    hc = mhc.HyperConnection(64, dynamic=dynamic, use_fused_weights=fused).to(DEV)
    H = torch.zeros((0, 5, 4, 64), device=DEV, dtype=torch.bfloat16, requires_grad=True)
    bo = torch.zeros((0, 5, 64), device=DEV, dtype=torch.bfloat16, requires_grad=True)
    # a dirty allocator pool: gradient buffers allocated next would hold these values
    junk = torch.full((1 << 20,), float("nan"), device=DEV)
    del junk
    bi, add = hc(H)
    Hn = add(bo)
    assert bi.shape == (0, 5, 64) and Hn.shape == (0, 5, 4, 64)
    (Hn.float().sum() + bi.float().sum()).backward()
    torch.cuda.synchronize()
    assert H.grad.shape == H.shape and bo.grad.shape == bo.shape
    for n, p in hc.named_parameters():
        assert p.grad is not None and float(p.grad.abs().sum()) == 0.0, n


# --------------------------------------------------------------------------- closure edge cases

def _oracle_grads(hc, H, bo, dHn, dbi):
    p = params_np(hc)
    _, _, cache = O.layer_forward(p, to_np(H), to_np(bo), hc.dynamic, True, hc.sinkhorn_iters, hc.eps)
    return O.layer_backward(p, cache, dHn, dbi)


def test_closure_called_twice():
    hc, H, bo, dHn, dbi = make_case(2, 16, 64, torch.float32, phi_std=0.05)
    Hl = H.clone().requires_grad_(True)
    bi, add = hc(Hl)
    bo2 = torch.randn_like(bo)
    Hn1, Hn2 = add(bo), add(bo2)
    torch.autograd.backward([Hn1, Hn2, bi], [dHn, dHn, dbi])
    g1 = _oracle_grads(hc, H, bo, to_np(dHn), to_np(dbi))
    g2 = _oracle_grads(hc, H, bo2, to_np(dHn), np.zeros_like(to_np(dbi)))
    # the loss is additive over the two closure outputs, so the gradient is the
    # sum of two single-call oracle gradients (the second with no branch_input term)
    assert rel_err(to_np(Hl.grad), g1["H"] + g2["H"]) < 1e-4
    assert rel_err(to_np(hc.phi.grad), g1["phi"] + g2["phi"]) < 1e-4


def test_closure_never_called_and_bi_only():
    hc, H, bo, dHn, dbi = make_case(2, 16, 64, torch.float32, phi_std=0.05)
    Hl = H.clone().requires_grad_(True)
    bi, _ = hc(Hl)
    bi.backward(dbi)
    g = _oracle_grads(hc, H, bo, np.zeros(H.shape), to_np(dbi))
    assert rel_err(to_np(Hl.grad), g["H"]) < 1e-4
    assert rel_err(to_np(hc.phi.grad), g["phi"]) < 1e-4
    assert rel_err(to_np(hc.H_post_base.grad), g["H_post_base"]) < 1e-4


@pytest.mark.parametrize("dynamic,fused", [(True, True), (False, True), (True, False)])
def test_partial_backward_then_branch_input_backward(dynamic, fused):
    """autograd.grad(H_new, branch_output) runs the closure's backward without node A's.  A later
    bi.backward() must then give the branch_input-only gradients: nothing of H_new's cotangent may
    reach dH or the parameter gradients."""
    hc, H, bo, dHn, dbi = make_case(2, 16, 64, torch.float32, dynamic=dynamic, fused=fused, phi_std=0.05,
                                    res_std=0.5)
    Hl = H.clone().requires_grad_(True)
    bol = bo.clone().requires_grad_(True)
    bi, add = hc(Hl)
    Hn = add(bol)
    (d_bo,) = torch.autograd.grad(Hn, bol, dHn, retain_graph=True)
    p = params_np(hc)
    _, _, cache = O.layer_forward(p, to_np(H), to_np(bo), dynamic, fused or not dynamic, hc.sinkhorn_iters, hc.eps)
    full = O.layer_backward(p, cache, to_np(dHn), to_np(dbi))
    assert rel_err(to_np(d_bo), full["bo"]) < 1e-4
    bi.backward(dbi)
    g = {k.replace(".weight", ""): v for k, v in O.layer_backward(p, cache, np.zeros(H.shape), to_np(dbi)).items()}
    assert rel_err(to_np(Hl.grad), g["H"]) < 1e-4
    for n, prm in hc.named_parameters():
        n = n.replace(".weight", "")
        assert rel_err(to_np(prm.grad).reshape(np.shape(g[n])), g[n]) < 1e-4, n


def test_closure_rejects_in_place_change_of_H():
    """add_residual recomputes H_res @ H from H, so an in-place change of H between forward and
    the call raises instead of mixing the new values (the reference's closure holds H_residual)."""
    hc, H, bo, _, _ = make_case(2, 16, 64, torch.float32, phi_std=0.05)
    Hc = H.clone()
    bi, add = hc(Hc)
    with torch.no_grad():
        Hc.add_(1.0)
    with pytest.raises(RuntimeError, match="modified in place"):
        add(bo)
    bi, add = hc(H)
    _, oHn, _ = O.layer_forward(params_np(hc), to_np(H), to_np(bo))
    assert rel_err(to_np(add(bo)), oHn) < 1e-5


def test_h_new_only_and_h_without_grad():
    hc, H, bo, dHn, dbi = make_case(2, 16, 64, torch.float32, phi_std=0.05)
    bol = bo.clone().requires_grad_(True)
    bi, add = hc(H)  # H does not require grad
    add(bol).backward(dHn)
    g = _oracle_grads(hc, H, bo, to_np(dHn), np.zeros(bo.shape))
    assert rel_err(to_np(bol.grad), g["bo"]) < 1e-4
    assert rel_err(to_np(hc.phi.grad), g["phi"]) < 1e-4
    assert rel_err(to_np(hc.alpha_res.grad), g["alpha_res"]) < 1e-4


def test_no_grad_forward_matches():
    hc, H, bo, dHn, dbi = make_case(2, 16, 64, torch.bfloat16, phi_std=0.02)
    with torch.no_grad():
        bi, add = hc(H)
        Hn = add(bo)
    obi, oHn, _ = O.layer_forward(params_np(hc), to_np(H), to_np(bo))
    assert rel_err(to_np(bi), obi) < 2e-2 and rel_err(to_np(Hn), oHn) < 2e-2


def test_state_dict_roundtrip_with_torch_baseline():
    import mhc

    hc = mhc.HyperConnection(64, layer_idx=3)
    ref = mhc.HyperConnectionTorch(64, layer_idx=3)
    ref.load_state_dict(hc.state_dict())
    assert set(hc.state_dict()) == set(ref.state_dict())


def test_training_steps_change_parameters():
    import mhc

    torch.manual_seed(42)
    hc = mhc.HyperConnection(dim=128, dynamic=True).to(DEV)
    layer = torch.nn.Linear(128, 128, device=DEV)
    opt = torch.optim.Adam(list(hc.parameters()) + list(layer.parameters()))
    init = {n: p.detach().clone() for n, p in hc.named_parameters()}
    for _ in range(3):
        opt.zero_grad()
        H = torch.randn(2, 32, 4, 128, device=DEV, requires_grad=True)
        bi, add = hc(H)
        add(layer(bi)).sum().backward()
        opt.step()
    changed = sum(1 for n, p in hc.named_parameters() if not torch.allclose(p, init[n]))
    assert changed > 0


@pytest.mark.parametrize("dynamic,fused,dtype", [(True, True, torch.float32), (True, True, torch.bfloat16),
                                                 (False, True, torch.float32), (True, False, torch.float32)])
def test_overridden_compute_weights_drives_forward(dynamic, fused, dtype):
    """A subclass that overrides _compute_weights changes the layer, as in the reference's forward
    (module.py:165-182): here it halves H_pre.  Outputs and every gradient match float64 torch
    autograd of the reference's composition with the halved H_pre."""
    import mhc
    from oracle import torch_path as TP

    class HalfPre(mhc.HyperConnection):
        def _compute_weights(self, H):
            H_post, H_pre, H_res = super()._compute_weights(H)
            return H_post, 0.5 * H_pre, H_res

    hc0, H, bo, dHn, dbi = make_case(2, 24, 64, dtype, dynamic=dynamic, fused=fused, phi_std=0.05, res_std=0.5)
    hc = HalfPre(64, dynamic=dynamic, use_fused_weights=fused).to(DEV)
    hc.load_state_dict(hc0.state_dict())
    bi, Hn, grads = run_gpu(hc, H, bo, dHn, dbi)

    leaves = {n: p.detach().double().cpu().requires_grad_(True) for n, p in hc.named_parameters()}
    Hl = H.detach().double().cpu().requires_grad_(True)
    bol = bo.detach().double().cpu().requires_grad_(True)
    H_post, H_pre, H_res = TP.layer_weights(leaves, Hl, dynamic, fused or not dynamic, hc.sinkhorn_iters, hc.eps)
    rbi, rhr = TP.stream_mix(Hl, 0.5 * H_pre, H_res)
    rHn = TP.add_residual(rhr, bol, H_post)
    torch.autograd.backward([rHn, rbi], [dHn.double().cpu(), dbi.double().cpu()])
    ftol, gtol = (1e-5, 1e-4) if dtype == torch.float32 else (2e-2, 2e-2)
    assert rel_err(to_np(bi), to_np(rbi)) < ftol and rel_err(to_np(Hn), to_np(rHn)) < ftol
    assert rel_err(to_np(grads["H"]), to_np(Hl.grad)) < gtol and rel_err(to_np(grads["bo"]), to_np(bol.grad)) < gtol
    for n, leaf in leaves.items():
        err = rel_err(to_np(grads[n.replace(".weight", "")]).reshape(leaf.shape), to_np(leaf.grad))
        assert err < 1e-4, (n, err)
    # the base class keeps the fused layer path: its branch_input uses the full H_pre
    bi0, _ = hc0(H)
    assert rel_err(to_np(bi), 0.5 * to_np(bi0)) < (1e-5 if dtype == torch.float32 else 2e-2)


def test_in_place_check_covers_views_of_one_buffer():
    """The closure's in-place check reads H's version counter, which every view of one storage
    shares: a write to another slice of the buffer H is a slice of also raises.  A clone of the
    slice is independent of the buffer."""
    hc, H, bo, _, _ = make_case(2, 16, 64, torch.float32, phi_std=0.05)
    buf = torch.stack([H, H])
    _, add = hc(buf[0])
    with torch.no_grad():
        buf[1].zero_()
    with pytest.raises(RuntimeError, match="modified in place"):
        add(bo)
    _, add = hc(buf[0].clone())
    with torch.no_grad():
        buf[1].zero_()
    _, oHn, _ = O.layer_forward(params_np(hc), to_np(H), to_np(bo))
    assert rel_err(to_np(add(bo)), oHn) < 1e-5


@pytest.mark.parametrize("dynamic,dtype", [(True, torch.bfloat16), (False, torch.float16), (True, torch.float32)])
def test_autocast_leaves_the_fused_layers_unchanged(dynamic, dtype):
    """Mixed-precision training runs the layer under torch.autocast.  The fused dynamic and static
    layers call no autocast-eligible torch op: every weight stays fp32 and the kernels see the same
    inputs, so the outputs and every gradient are the same bits as without autocast (as in the
    reference, whose fused path is Triton launches on the same tensors)."""
    hc, H, bo, dHn, dbi = make_case(3, 40, 96, dtype, dynamic=dynamic, phi_std=0.02, res_std=0.5)
    bi0, Hn0, g0 = run_gpu(hc, H, bo, dHn, dbi)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        bi1, Hn1, g1 = run_gpu(hc, H, bo, dHn, dbi)
    assert bi1.dtype == dtype and Hn1.dtype == dtype
    assert torch.equal(bi0, bi1) and torch.equal(Hn0, Hn1)
    for n in g0:
        assert torch.equal(g0[n], g1[n]), n


@pytest.mark.parametrize("dynamic,fused", [(True, True), (False, True), (True, False)])
@pytest.mark.parametrize("use_reentrant", [False, True])
def test_activation_checkpointing(dynamic, fused, use_reentrant):
    """A transformer block under torch.utils.checkpoint: the layer's forward runs again inside the
    backward.  The kernels are deterministic, so every gradient is the same bits as the same block
    without checkpointing."""
    from torch.utils.checkpoint import checkpoint

    hc, H, _, dHn, _ = make_case(2, 24, 64, torch.bfloat16, dynamic=dynamic, fused=fused, phi_std=0.02,
                                 res_std=0.5)
    torch.manual_seed(3)
    branch = torch.nn.Linear(64, 64, device=DEV).to(torch.bfloat16)

    def block(h):
        bi, add = hc(h)
        return add(branch(bi))

    def grads(ckpt):
        hc.zero_grad(set_to_none=True)
        branch.zero_grad(set_to_none=True)
        Hl = H.clone().requires_grad_(True)
        out = checkpoint(block, Hl, use_reentrant=use_reentrant) if ckpt else block(Hl)
        out.backward(dHn)
        g = {n: p.grad.clone() for n, p in list(hc.named_parameters()) + list(branch.named_parameters())}
        g["H"] = Hl.grad
        return out.detach(), g

    out0, g0 = grads(False)
    out1, g1 = grads(True)
    assert torch.equal(out0, out1)
    assert set(g0) == set(g1)
    for n in g0:
        assert torch.equal(g0[n], g1[n]), n


@pytest.mark.parametrize("dynamic", [True, False])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_module_cast_to_half_precision(dynamic, dtype):
    """The reference's benchmark casts the whole module with .half() (benchmarks/benchmark.py:147,150).
    The kernels read the half-precision parameters as fp32 values, so the layer is the oracle's
    at those parameter values; every parameter gradient comes back in the parameter's dtype,
    rounded once from fp32 (to within one unit in the last place of its largest entry)."""
    hc, H, bo, dHn, dbi = make_case(2, 48, 96, dtype, dynamic=dynamic, phi_std=0.02, res_std=0.5)
    hc = hc.to(dtype)
    bi, Hn, grads = run_gpu(hc, H, bo, dHn, dbi)
    p = params_np(hc)
    obi, oHn, cache = O.layer_forward(p, to_np(H), to_np(bo), dynamic, True, hc.sinkhorn_iters, hc.eps)
    og = {k.replace(".weight", ""): v for k, v in O.layer_backward(p, cache, to_np(dHn), to_np(dbi)).items()}
    assert rel_err(to_np(bi), obi) < 2e-2 and rel_err(to_np(Hn), oHn) < 2e-2
    assert rel_err(to_np(grads["H"]), og["H"]) < 2e-2 and rel_err(to_np(grads["bo"]), og["bo"]) < 2e-2
    ulp = 2.0 ** -10 if dtype == torch.float16 else 2.0 ** -7
    for n, param in hc.named_parameters():
        k = n.replace(".weight", "")
        assert grads[k].dtype == param.dtype == dtype, n
        err = rel_err(to_np(grads[k]).reshape(np.shape(og[k])), og[k])
        assert err < ulp, (n, err)


@pytest.mark.parametrize("dynamic,fused", [(True, True), (False, True), (True, False)])
def test_inference_mode(dynamic, fused):
    """Serving stacks run under torch.inference_mode, where new tensors are inference tensors with
    no version counter.  The layer runs there (the closure's in-place check is skipped for such an
    H) and gives the same bits as under torch.no_grad; so do the four public ops."""
    import mhc

    hc, H, bo, _, _ = make_case(3, 20, 64, torch.bfloat16, dynamic=dynamic, fused=fused, phi_std=0.02,
                                res_std=0.5)
    with torch.no_grad():
        bi0, add0 = hc(H)
        Hn0 = add0(bo)
    with torch.inference_mode():
        Hi, boi = H.clone(), bo.clone()
        assert Hi.is_inference()
        bi1, add1 = hc(Hi)
        Hn1 = add1(boi)
        # a normal tensor made before inference mode keeps its check
        bi2, add2 = hc(H)
        Hn2 = add2(bo)
    assert torch.equal(bi0, bi1) and torch.equal(Hn0, Hn1)
    assert torch.equal(bi0, bi2) and torch.equal(Hn0, Hn2)
    Hc = H.clone()
    with torch.inference_mode():
        _, add3 = hc(Hc)
        Hc.add_(1.0)
        with pytest.raises(RuntimeError, match="modified in place"):
            add3(bo)
    if dynamic and fused:
        x = H.float().mean(1).reshape(3, -1)
        bias = torch.cat([hc.H_pre_base, hc.H_post_base, hc.H_res_base.flatten()]).detach()
        alphas = (hc.alpha_pre, hc.alpha_post, hc.alpha_res)

        def ops(x, H, bo):
            pre, post, res = mhc.fused_dynamic_weights(x, hc.phi, bias, *alphas, 20, 1e-6)
            bi, h_res = mhc.fused_stream_mix(H, pre, res)
            return pre, post, res, bi, h_res, mhc.fused_add_residual(h_res, bo, post), mhc.sinkhorn_knopp(res, 20)

        with torch.no_grad():
            want = ops(x, H, bo)
        with torch.inference_mode():
            got = ops(x.clone(), H.clone(), bo.clone())
        for a, b in zip(want, got):
            assert torch.equal(a, b)


@pytest.mark.parametrize("dynamic,fused", [(True, True), (False, True), (True, False)])
def test_frozen_parameters(dynamic, fused):
    """Fine-tuning with the layer's parameters frozen (all of them, or only the first): dH and
    d branch_output, and the gradients of the parameters left trainable, are the same bits as with
    every parameter trainable; frozen parameters get no gradient."""
    hc, H, bo, dHn, dbi = make_case(2, 24, 64, torch.bfloat16, dynamic=dynamic, fused=fused, phi_std=0.02,
                                    res_std=0.5)
    _, _, g_all = run_gpu(hc, H, bo, dHn, dbi)
    names = [n for n, _ in hc.named_parameters()]
    for frozen in (names, names[:1]):
        for n, p in hc.named_parameters():
            p.requires_grad_(n not in frozen)
        _, _, g = run_gpu(hc, H, bo, dHn, dbi)
        assert torch.equal(g["H"], g_all["H"]) and torch.equal(g["bo"], g_all["bo"])
        for n in names:
            k = n.replace(".weight", "")
            if n in frozen:
                assert g[k] is None, n
            else:
                assert torch.equal(g[k], g_all[k]), n
    for p in hc.parameters():
        p.requires_grad_(True)


def _offset_by_one(t):
    """A contiguous copy of t that starts one element past a 16-byte boundary."""
    buf = torch.empty(t.numel() + 8, dtype=t.dtype, device=t.device)
    out = buf[1:1 + t.numel()].view(t.shape)
    out.copy_(t)
    return out


@pytest.mark.parametrize("B,S,D,dynamic,fused", [(2, 24, 64, True, True), (2, 24, 64, False, True),
                                                 (2, 24, 64, True, False), (64, 1, 64, True, True),
                                                 (64, 2, 8192, True, True)])
def test_contiguous_inputs_off_a_16_byte_boundary(B, S, D, dynamic, fused):
    """H and branch_output contiguous but one element off a 16-byte boundary (slices of a packed
    buffer): every kernel that loads 16 bytes at a time checks the pointers it is given and the
    layer takes the element-wise forms, on the small-batch and the bulk-batch paths.  Against the
    oracle."""
    hc, H, bo, dHn, dbi = make_case(B, S, D, torch.bfloat16, dynamic=dynamic, fused=fused, phi_std=0.02,
                                    res_std=0.5)
    dHnm, dbim = _offset_by_one(dHn), _offset_by_one(dbi)
    assert _offset_by_one(H).data_ptr() % 16 != 0 and _offset_by_one(H).is_contiguous()
    check_layer(hc, H, bo, dHnm, dbim, 2e-2, 2e-2, 1e-4, copy=_offset_by_one)
