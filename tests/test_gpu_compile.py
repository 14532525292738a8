"""torch.compile over the HIP path, and torch.library.opcheck of every registered op.

Compiled (``fullgraph=True``: any graph break fails the test) and eager runs of
the same step launch the same kernels in the same order, so outputs and every
gradient must agree bit for bit.  The compiled layer hands the closure's
gradients to node A through a link output, as the eager layer does.
``aot_eager`` runs the traced graph with torch's own kernels around the
``torch.ops.mhc`` nodes; the default backend (inductor) generates its own
kernels for the glue around them.  Compiled steps with an independent
branch_output are also checked against the float64 oracle layer.
"""

import numpy as np
import pytest
import torch

import mhc
from helpers import rel_err, to_np
from oracle import mhc_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _compile(fn, dynamic=False, backend="aot_eager"):
    torch._dynamo.reset()
    if backend == "inductor":
        return torch.compile(fn, fullgraph=True, dynamic=dynamic)
    return torch.compile(fn, backend=backend, fullgraph=True, dynamic=dynamic)


def _layer_case(dynamic, fused, dtype, B=2, S=64, D=256, seed=0):
    g = torch.Generator().manual_seed(seed)
    hc = mhc.HyperConnection(D, dynamic=dynamic, use_fused_weights=fused, layer_idx=1)
    with torch.no_grad():
        if dynamic and fused:
            hc.phi.copy_(torch.randn(hc.phi.shape, generator=g) * 0.02)
        if dynamic and not fused:
            for lin in (hc.W_pre, hc.W_post, hc.W_res):
                lin.weight.copy_(torch.randn(lin.weight.shape, generator=g) * 0.02)
        hc.H_res_base.add_(torch.randn((4, 4), generator=g) * 0.5)
    H = torch.randn((B, S, 4, D), generator=g).to(dtype)
    W = torch.randn((D, D), generator=g) / D ** 0.5
    gHn = torch.randn((B, S, 4, D), generator=g).to(dtype)
    gbi = torch.randn((B, S, D), generator=g).to(dtype)
    return hc.to(DEV), H.to(DEV), W.to(DEV), gHn.to(DEV), gbi.to(DEV)


def _run(step, hc, H, W, gHn, gbi, calls):
    hc.zero_grad(set_to_none=True)
    Hl = H.clone().requires_grad_(True)
    Wl = W.clone().requires_grad_(True)
    outs = step(Hl, Wl)
    grads = [gbi] + [gHn * (k + 1) for k in range(calls)]
    torch.autograd.backward(list(outs), grads)
    res = {"out%d" % i: o.detach() for i, o in enumerate(outs)}
    res["H"] = Hl.grad
    res["W"] = Wl.grad
    for n, p in hc.named_parameters():
        res[n] = p.grad
    return res


def _assert_identical(a, b):
    assert a.keys() == b.keys()
    for k in a:
        if a[k] is None or b[k] is None:
            assert a[k] is None and b[k] is None, k
            continue
        assert a[k].dtype == b[k].dtype and a[k].shape == b[k].shape, k
        assert torch.equal(a[k], b[k]), (k, float((a[k].float() - b[k].float()).abs().max()))


@pytest.mark.parametrize("dtype,calls", [(torch.bfloat16, 1), (torch.bfloat16, 0), (torch.bfloat16, 2),
                                         (torch.float32, 1)])
@pytest.mark.parametrize("dynamic,fused", [(True, True), (False, True), (True, False)])
def test_compiled_layer_step_matches_eager_bitwise(dynamic, fused, dtype, calls):
    hc, H, W, gHn, gbi = _layer_case(dynamic, fused, dtype)

    def step(Hl, Wl):
        bi, add = hc(Hl)
        outs = [bi]
        for k in range(calls):
            bo = torch.tanh(bi.float() @ Wl * (k + 1)).to(bi.dtype)  # the caller's layer
            outs.append(add(bo))
        return outs

    eager = _run(step, hc, H, W, gHn, gbi, calls)
    compiled = _run(_compile(step), hc, H, W, gHn, gbi, calls)
    _assert_identical(eager, compiled)
    assert eager["H"] is not None and torch.isfinite(eager["H"].float()).all()


@pytest.mark.parametrize("backend", ["aot_eager", "inductor"])
@pytest.mark.parametrize("dynamic,fused,dtype", [(True, True, torch.bfloat16), (True, True, torch.float32),
                                                 (False, True, torch.float32), (True, False, torch.float32)])
def test_compiled_layer_step_matches_oracle_and_eager(dynamic, fused, dtype, backend):
    """bi, add = hc(H); H_new = add(bo) with bo an independent leaf, compiled (fullgraph) with
    aot_eager and with the default inductor backend: bit-identical to eager, and within the
    stated tolerances of the float64 oracle layer (fp32: 1e-5 forward, 1e-4 gradients; bf16:
    2e-2 outputs, 1e-4 parameter gradients)."""
    hc, H, _, gHn, gbi = _layer_case(dynamic, fused, dtype)
    g = torch.Generator().manual_seed(7)
    bo = torch.randn(gbi.shape, generator=g).to(dtype).to(DEV)

    def step(Hl, bol):
        bi, add = hc(Hl)
        return bi, add(bol)

    def run(f):
        hc.zero_grad(set_to_none=True)
        Hl, bol = H.clone().requires_grad_(True), bo.clone().requires_grad_(True)
        bi, Hn = f(Hl, bol)
        torch.autograd.backward([bi, Hn], [gbi, gHn])
        out = {"bi": bi.detach(), "H_new": Hn.detach(), "H": Hl.grad, "bo": bol.grad}
        out.update({n.replace(".weight", ""): p.grad for n, p in hc.named_parameters()})
        return out

    eager = run(step)
    compiled = run(_compile(step, backend=backend))
    if backend == "inductor" and dynamic and not fused:
        # The unfused weights come from torch ops (RMS, Linear, sigmoid) that inductor fuses
        # into kernels of its own, rounded differently in the last bits than eager's.
        for k in eager:
            assert rel_err(to_np(compiled[k]), to_np(eager[k])) < 1e-5, k
    else:
        _assert_identical(eager, compiled)
    p = {n.replace(".weight", ""): to_np(v) for n, v in hc.named_parameters()}
    obi, oHn, cache = O.layer_forward(p, to_np(H), to_np(bo), dynamic, fused or not dynamic, hc.sinkhorn_iters,
                                      hc.eps)
    og = {k.replace(".weight", ""): v for k, v in O.layer_backward(p, cache, to_np(gHn), to_np(gbi)).items()}
    ftol, gtol = (1e-5, 1e-4) if dtype == torch.float32 else (2e-2, 2e-2)
    ptol = 1e-4
    assert rel_err(to_np(compiled["bi"]), obi) < ftol and rel_err(to_np(compiled["H_new"]), oHn) < ftol
    assert rel_err(to_np(compiled["H"]), og["H"]) < gtol and rel_err(to_np(compiled["bo"]), og["bo"]) < gtol
    for n in p:
        assert rel_err(to_np(compiled[n]).reshape(np.shape(og[n])), og[n]) < ptol, n


def _step_of(hc):
    def step(Hl, Wl):
        bi, add = hc(Hl)
        return [bi, add(torch.tanh(bi.float() @ Wl).to(bi.dtype))]
    return step


@pytest.mark.parametrize("dynamic,fused", [(True, True), (False, True), (True, False)])
def test_compiled_reduce_overhead_matches_eager(dynamic, fused):
    """torch.compile(mode="reduce-overhead"): inductor replays the step, forward and backward, as
    CUDA graphs from its own memory pool, workspaces included.  Four steps with new input values:
    each one the same bits as the eager step (bo an independent leaf, so that no torch op of the
    caller's, which inductor would compile differently, sits between the two halves of the layer;
    the unfused weights are such torch ops: within 1e-5 in fp32, two bf16 units in the last place
    in the bf16 outputs and dH)."""
    hc, H, _, gHn, gbi = _layer_case(dynamic, fused, torch.bfloat16)
    g = torch.Generator().manual_seed(7)
    bo = torch.randn(gbi.shape, generator=g).to(torch.bfloat16).to(DEV)

    def step(Hl, bol):
        bi, add = hc(Hl)
        return bi, add(bol)

    def run(f, Hs):
        hc.zero_grad(set_to_none=True)
        Hl, bol = Hs.clone().requires_grad_(True), bo.clone().requires_grad_(True)
        bi, Hn = f(Hl, bol)
        torch.autograd.backward([bi, Hn], [gbi, gHn])
        out = {"bi": bi.detach().clone(), "H_new": Hn.detach().clone(), "H": Hl.grad, "bo": bol.grad}
        out.update({n: p.grad.clone() for n, p in hc.named_parameters()})
        return out

    torch._dynamo.reset()
    step_c = torch.compile(step, mode="reduce-overhead", fullgraph=True)
    for it in range(4):
        Hs = (H.float() * (1 + 0.25 * it)).to(H.dtype)
        want = run(step, Hs)
        torch.compiler.cudagraph_mark_step_begin()
        got = run(step_c, Hs)
        if dynamic and not fused:
            # fp32 results to 1e-5; the bf16 ones (bi, H_new, dH, d_bo) to two units in the last
            # place, where the weights' last fp32 bits move a rounding
            for k in want:
                tol = 1e-5 if want[k].dtype == torch.float32 else 2.0 ** -6
                assert rel_err(to_np(got[k]), to_np(want[k])) < tol, (it, k)
        else:
            _assert_identical(want, got)


def test_compiled_layer_with_dynamic_shapes():
    """One compiled graph serves three sequence lengths (symbolic shapes through the fake kernels)."""
    from torch._dynamo.utils import counters

    hc, H, W, gHn, gbi = _layer_case(True, True, torch.bfloat16, S=96)
    step = _step_of(hc)
    step_c = _compile(step, dynamic=True)
    counters.clear()
    for S in (64, 96, 33):
        case = (H[:, :S].contiguous(), W, gHn[:, :S].contiguous(), gbi[:, :S].contiguous())
        _assert_identical(_run(step, hc, *case, 1), _run(step_c, hc, *case, 1))
    assert counters["stats"]["unique_graphs"] == 1


@pytest.mark.parametrize("backend", ["aot_eager", "inductor"])
@pytest.mark.parametrize("dynamic,fused", [(True, True), (False, True), (True, False)])
def test_compiled_layer_with_strided_h(dynamic, fused, backend):
    """A strided H under torch.compile: the traced forward makes it contiguous once; outputs and
    gradients (returned in H's own strides) match eager bit for bit and the float64 oracle."""
    hc, H, _, gHn, gbi = _layer_case(dynamic, fused, torch.float32, S=40, D=128)
    bo = torch.randn(gbi.shape, generator=torch.Generator().manual_seed(9)).to(DEV)
    Ht = H.permute(0, 1, 3, 2).contiguous().permute(0, 1, 3, 2)
    assert not Ht.is_contiguous() and torch.equal(Ht, H)

    def step(Hl, bol):
        bi, add = hc(Hl)
        return bi, add(bol)

    def run(f):
        hc.zero_grad(set_to_none=True)
        Hl, bol = Ht.detach().requires_grad_(True), bo.clone().requires_grad_(True)
        bi, Hn = f(Hl, bol)
        torch.autograd.backward([bi, Hn], [gbi, gHn])
        assert Hl.grad.shape == Hl.shape
        out = {"bi": bi.detach(), "H_new": Hn.detach(), "H": Hl.grad.contiguous(), "bo": bol.grad}
        out.update({n.replace(".weight", ""): p.grad for n, p in hc.named_parameters()})
        return out

    eager = run(step)
    compiled = run(_compile(step, backend=backend))
    if backend == "inductor" and not fused:
        for k in eager:
            assert rel_err(to_np(compiled[k]), to_np(eager[k])) < 1e-5, k
    else:
        _assert_identical(eager, compiled)
    p = {n.replace(".weight", ""): to_np(v) for n, v in hc.named_parameters()}
    obi, oHn, cache = O.layer_forward(p, to_np(H), to_np(bo), dynamic, fused or not dynamic, hc.sinkhorn_iters,
                                      hc.eps)
    og = {k.replace(".weight", ""): v for k, v in O.layer_backward(p, cache, to_np(gHn), to_np(gbi)).items()}
    assert rel_err(to_np(compiled["bi"]), obi) < 1e-5 and rel_err(to_np(compiled["H_new"]), oHn) < 1e-5
    assert rel_err(to_np(compiled["H"]), og["H"]) < 1e-4 and rel_err(to_np(compiled["bo"]), og["bo"]) < 1e-4
    for n in p:
        assert rel_err(to_np(compiled[n]).reshape(np.shape(og[n])), og[n]) < 1e-4, n


@pytest.mark.parametrize("backend", ["aot_eager", "inductor"])
@pytest.mark.parametrize("dynamic,fused", [(True, True), (False, True), (True, False)])
def test_compiled_closure_reads_h_as_it_was_at_forward(dynamic, fused, backend):
    """H changed in place between forward and the closure call, inside a compiled function: the
    closure mixes H as it was at forward time (the reference's closure holds H_residual,
    module.py:177-180), and the change itself still reaches H.  Eager raises instead; traced code
    cannot read a version counter, so the traced layer takes a snapshot of H."""
    hc, H, _, _, gbi = _layer_case(dynamic, fused, torch.float32, S=32, D=128)
    bo = torch.randn(gbi.shape, generator=torch.Generator().manual_seed(11)).to(DEV)

    def step(Hm, bol):
        bi, add = hc(Hm)
        Hm.mul_(2.0)
        return bi, add(bol)

    Hm = H.clone()
    with torch.no_grad():
        bi, Hn = _compile(step, backend=backend)(Hm, bo)
    assert torch.equal(Hm, 2.0 * H)
    obi, oHn, _ = O.layer_forward({n.replace(".weight", ""): to_np(v) for n, v in hc.named_parameters()},
                                  to_np(H), to_np(bo), dynamic, fused or not dynamic, hc.sinkhorn_iters, hc.eps)
    assert rel_err(to_np(bi), obi) < 1e-5 and rel_err(to_np(Hn), oHn) < 1e-5


def test_compiled_public_ops_match_eager_bitwise():
    g = torch.Generator().manual_seed(1)
    B, S, D = 2, 32, 128
    H = torch.randn((B, S, 4, D), generator=g).bfloat16().to(DEV)
    x = torch.randn((B, 4 * D), generator=g).to(DEV)
    phi = (torch.randn((4 * D, 24), generator=g) * 0.05).to(DEV)
    bias = torch.randn(24, generator=g).to(DEV)
    alphas = [torch.tensor([0.3], device=DEV), torch.tensor([0.2], device=DEV), torch.tensor([0.1], device=DEV)]
    M = torch.exp(torch.randn((64, 4, 4), generator=g)).to(DEV)
    bo = torch.randn((B, S, D), generator=g).bfloat16().to(DEV)

    def fn(H, x, phi, bias, a0, a1, a2, M, bo):
        pre, post, res = mhc.fused_dynamic_weights(x, phi, bias, a0, a1, a2)
        bi, hres = mhc.fused_stream_mix(H, pre, res)
        Hn = mhc.fused_add_residual(hres, bo * bi, post)
        P = mhc.sinkhorn_knopp(M, 20)
        return Hn.float().square().mean() + P.square().sum() + bi.float().mean()

    def run(f):
        leaves = [t.clone().requires_grad_(True) for t in (H, x, phi, bias, *alphas, M, bo)]
        loss = f(*leaves)
        loss.backward()
        return {"loss": loss.detach(), **{"g%d" % i: t.grad for i, t in enumerate(leaves)}}

    _assert_identical(run(fn), run(_compile(fn)))


def test_compiled_model_ends_match_eager_bitwise():
    """expand -> two HyperConnection layers -> collapse, compiled as one graph."""
    from mhc.streams import collapse_streams, expand_streams

    g = torch.Generator().manual_seed(4)
    B, S, D = 2, 48, 128
    hcs = [mhc.HyperConnection(D, layer_idx=i).to(DEV) for i in range(2)]
    with torch.no_grad():
        for hc in hcs:
            hc.phi.copy_((torch.randn(hc.phi.shape, generator=g) * 0.02).to(DEV))
    x = torch.randn((B, S, D), generator=g).bfloat16().to(DEV)
    W = (torch.randn((D, D), generator=g) / D ** 0.5).to(DEV)
    gy = torch.randn((B, S, D), generator=g).bfloat16().to(DEV)

    def model(xl, Wl):
        H = expand_streams(xl)
        for hc in hcs:
            bi, add = hc(H)
            H = add(torch.tanh(bi.float() @ Wl).to(bi.dtype))
        return collapse_streams(H)

    def run(f):
        for hc in hcs:
            hc.zero_grad(set_to_none=True)
        xl, Wl = x.clone().requires_grad_(True), W.clone().requires_grad_(True)
        y = f(xl, Wl)
        y.backward(gy)
        out = {"y": y.detach(), "x": xl.grad, "W": Wl.grad}
        for i, hc in enumerate(hcs):
            out.update({f"{i}.{n}": p.grad for n, p in hc.named_parameters()})
        return out

    _assert_identical(run(model), run(_compile(model)))


_CASES = []


def _opcheck_cases():
    if _CASES:
        return _CASES
    g = torch.Generator().manual_seed(2)
    B, S, D, R, K = 2, 16, 64, 3, 256
    r = lambda *s, dt=torch.float32: torch.randn(s, generator=g).to(dt).to(DEV)  # noqa: E731
    H, bi, bo = r(B, S, 4, D, dt=torch.bfloat16), r(B, S, D, dt=torch.bfloat16), r(B, S, D, dt=torch.bfloat16)
    pre = torch.softmax(r(B, 4), -1)
    post = torch.sigmoid(r(B, 4)) * 2
    M = torch.exp(r(5, 4, 4))
    res = mhc.sinkhorn_knopp(M[:B].clone(), 20)
    a = [torch.tensor([0.1], device=DEV) for _ in range(3)]
    x, phi, bias = r(R, K), r(K, 24) * 0.02, r(24)
    Hp, Hpo, Hr, aux = torch.ops.mhc.dynamic_weights_forward(x, phi, bias, *a, 20, 1e-6)
    base = [r(4), r(4), r(4, 4)]
    phiL = r(4 * D, 24) * 0.02
    biL, xL, wL, auxL = torch.ops.mhc.layer_dynamic_forward(H, phiL, *base, *a, 20, 1e-6)
    _, wS = torch.ops.mhc.layer_static_forward(H, *base, 20)
    dpost = r(B, 4)
    rg = lambda t: t.clone().requires_grad_(True)  # noqa: E731
    _CASES.extend([
        ("sinkhorn_forward", (rg(M), 20, 1e-8)),
        ("sinkhorn_backward", (M, r(5, 4, 4), 20, 1e-8)),
        ("stream_mix_forward", (rg(H.float()), rg(pre), rg(res))),
        ("stream_mix_backward", (bi, H, H, pre, res)),
        ("add_residual_forward", (rg(H.float()), rg(bo.float()), rg(post))),
        ("add_residual_backward", (H, bo, post)),
        ("dynamic_weights_forward", (rg(x), rg(phi), rg(bias), *[rg(t) for t in a], 20, 1e-6)),
        ("dynamic_weights_backward", (x, phi, bias, *a, aux, Hp, r(R, 4), None, r(R, 4, 4), 20, 1e-6)),
        ("mean_pool", (rg(H.float()),)),
        ("layer_dynamic_forward", (H, phiL, *base, *a, 20, 1e-6)),
        ("layer_dynamic_backward", (H, bi, H, dpost, phiL, *base, *a, xL, wL, auxL, 20, 1e-6)),
        ("layer_dynamic_backward", (H, bi, None, None, phiL, *base, *a, xL, wL, auxL, 20, 1e-6)),
        ("layer_static_forward", (H, *base, 20)),
        ("layer_static_backward", (H, bi, H, dpost, *base, wS, 20)),
        ("layer_branch_input", (H, wL)),
        ("layer_mix_backward", (H, bi, H, wL)),
        ("layer_mix_reduce", (H, bi, H, wL)),
        ("layer_mix_reduce", (H, None, None, wL)),
        ("layer_mix_dh", (bi, H, wL, xL, H)),
        ("layer_mix_dh", (None, None, wL, None, H)),
        ("layer_add_forward", (H, bo, wL)),
        ("layer_add_backward", (H, bo, wL)),
        ("stream_expand", (rg(bo.float()), 0.5, torch.bfloat16)),
        ("stream_collapse", (rg(H.float()), 0.25, None)),
    ])
    return _CASES


N_CASES = 24


def test_opcheck_covers_every_registered_op():
    cases = _opcheck_cases()
    assert len(cases) == N_CASES
    assert {n for n, _ in cases} == {n for n in dir(torch.ops.mhc) if not n.startswith("_") and n != "name"}


@pytest.mark.parametrize("idx", range(N_CASES))
def test_opcheck(idx):
    """Schema (no mutation, no aliasing), fake kernel against the real one (shapes,
    dtypes, strides), autograd registration and AOT dispatch with dynamic shapes."""
    name, args = _opcheck_cases()[idx]
    print(f"opcheck mhc::{name}", flush=True)
    torch.library.opcheck(getattr(torch.ops.mhc, name).default, args)
