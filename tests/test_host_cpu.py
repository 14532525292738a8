"""Host logic that needs no GPU: module construction / parameters / init
(reference src/mhc/module.py:37-101,191-224), the public API surface, the
pure-PyTorch baselines on CPU, and the layer's node-B -> node-A gradient wiring
(run on float64 oracle stand-ins for the HIP launchers)."""

import numpy as np
import pytest
import torch

import mhc
from mhc import _layer
from oracle import mhc_oracle as O


def test_public_api_surface():
    assert mhc.__all__ == [
        "HyperConnection", "sinkhorn_knopp", "fused_stream_mix", "fused_add_residual", "fused_dynamic_weights",
        "sinkhorn_knopp_torch", "fused_stream_mix_torch", "fused_add_residual_torch",
        "fused_dynamic_weights_torch", "HyperConnectionTorch",
    ]
    assert mhc.__version__ == "0.1.0"


def test_parameters_and_init_match_reference_layout():
    hc = mhc.HyperConnection(16, layer_idx=6)
    shapes = {n: tuple(p.shape) for n, p in hc.named_parameters()}
    assert shapes == {"H_post_base": (4,), "H_pre_base": (4,), "H_res_base": (4, 4), "phi": (64, 24),
                      "alpha_pre": (1,), "alpha_post": (1,), "alpha_res": (1,)}
    assert torch.equal(hc.H_pre_base.data, torch.tensor([0.0, 0, 1, 0]))  # 6 % 4 == 2
    assert torch.equal(hc.H_res_base.data, torch.eye(4))
    assert torch.equal(hc.H_post_base.data, torch.ones(4))
    assert hc.alpha_res.item() == np.float32(0.1)
    with torch.no_grad():
        for p in hc.parameters():
            p.add_(1.0)
    hc.init_weights(layer_idx=1)
    assert torch.equal(hc.H_pre_base.data, torch.tensor([0.0, 1, 0, 0]))
    assert torch.count_nonzero(hc.phi).item() == 0
    assert "use_fused_weights=True" in repr(hc)
    un = mhc.HyperConnection(16, use_fused_weights=False)
    assert {n for n, _ in un.named_parameters()} == {
        "H_post_base", "H_pre_base", "H_res_base", "W_post.weight", "W_pre.weight", "W_res.weight",
        "scale_post", "scale_pre", "scale_res"}
    st = mhc.HyperConnection(16, dynamic=False)
    assert not st.use_fused_weights and {n for n, _ in st.named_parameters()} == {
        "H_post_base", "H_pre_base", "H_res_base"}


def test_state_dict_compatible_with_torch_baseline():
    for kw in ({}, {"use_fused_weights": False}, {"dynamic": False}):
        a = mhc.HyperConnection(32, **kw)
        b = mhc.HyperConnectionTorch(32, **kw)
        b.load_state_dict(a.state_dict())


def test_torch_baselines_run_on_cpu_with_autograd():
    hc = mhc.HyperConnectionTorch(16)
    H = torch.randn(2, 8, 4, 16, requires_grad=True)
    bi, add = hc(H)
    add(torch.randn(2, 8, 16)).sum().backward()
    assert H.grad.shape == H.shape and hc.phi.grad is not None


class _OracleLaunchers:
    """float64 oracle stand-ins for the static layer's launchers, so the autograd wiring of
    _layer's two nodes (node B's gradients reaching node A through the link and w) can run
    on the CPU.  Only this test installs them."""

    @staticmethod
    def static_forward(H, pre, post, res, iters):
        B = H.shape[0]
        Hp, Hq, Hr = O.static_weights(pre.detach().numpy(), post.detach().numpy(), res.detach().numpy(), B, iters)
        bi, _ = O.stream_mix(H.detach().numpy(), Hq, Hr)
        w = np.concatenate([Hq, Hp, Hr.reshape(B, 16)], axis=1)
        return torch.tensor(bi), torch.tensor(w)

    @staticmethod
    def static_backward(H, d_bi, dH_new, dH_post, pre, post, res, w, iters, need_dH=True):
        B, S, _, D = H.shape
        wn = w.detach().numpy()
        d_bi = np.zeros((B, S, D)) if d_bi is None else d_bi.numpy()
        dHn = np.zeros((B, S, 4, D)) if dH_new is None else dH_new.numpy()
        dpost = np.zeros((B, 4)) if dH_post is None else dH_post.numpy()
        dH, dpre, dres = O.stream_mix_backward(d_bi, dHn, H.detach().numpy(), wn[:, 0:4], wn[:, 8:].reshape(B, 4, 4))
        gq, gp, gr = O.static_weights_backward(pre.detach().numpy(), post.detach().numpy(), res.detach().numpy(),
                                               dpost, dpre, dres, iters)
        return (torch.tensor(dH) if need_dH else None), torch.tensor(np.concatenate([gq, gp, gr.reshape(16)]))

    @staticmethod
    def add_forward(H, bo, w):
        B = H.shape[0]
        wn = w.detach().numpy()
        _, hr = O.stream_mix(H.detach().numpy(), wn[:, 0:4], wn[:, 8:].reshape(B, 4, 4))
        return torch.tensor(O.add_residual(hr, bo.detach().numpy(), wn[:, 4:8]))

    @staticmethod
    def add_backward(dH_new, bo, w):
        _, d_bo, dpost = O.add_residual_backward(dH_new.numpy(), bo.detach().numpy(), w.detach().numpy()[:, 4:8])
        return torch.tensor(d_bo), torch.tensor(dpost)


class _UnfusedLaunchers:
    """float64 oracle stand-ins for the launchers of the unfused dynamic layer (the sequence-mean
    node that writes dH, node A's reductions, the closure), so that the pool node's wiring runs on
    the CPU: dH_new, d_branch_input and w must reach it through the links, and grad_x / S must
    land in dH once.  torch's Sinkhorn stands in for the HIP one."""

    @staticmethod
    def mean_pool(H):
        B, S, n, D = H.shape
        return H.detach().mean(dim=1).reshape(B, n * D)

    @staticmethod
    def branch_input(H, w):
        B = H.shape[0]
        wn = w.detach().numpy()
        bi, _ = O.stream_mix(H.detach().numpy(), wn[:, 0:4], wn[:, 8:].reshape(B, 4, 4))
        return torch.tensor(bi)

    @staticmethod
    def mix_backward(H, d_bi, dH_new, w, need_dH=True):
        B, S, _, D = H.shape
        wn = w.detach().numpy()
        d_bi = np.zeros((B, S, D)) if d_bi is None else d_bi.numpy()
        dHn = np.zeros((B, S, 4, D)) if dH_new is None else dH_new.numpy()
        dH, dpre, dres = O.stream_mix_backward(d_bi, dHn, H.detach().numpy(), wn[:, 0:4], wn[:, 8:].reshape(B, 4, 4))
        return (torch.tensor(dH) if need_dH else None), torch.tensor(dpre), torch.tensor(dres.reshape(B, 16))

    @staticmethod
    def mix_dh(d_bi, dH_new, w, grad_x, H_shape, h_dtype):
        B, S, _, D = H_shape
        wn = w.detach().numpy()
        d_bi = np.zeros((B, S, D)) if d_bi is None else d_bi.numpy()
        dHn = np.zeros((B, S, 4, D)) if dH_new is None else dH_new.numpy()
        gx = np.zeros((B, 4 * D)) if grad_x is None else grad_x.numpy()
        dH, _, _ = O.stream_mix_backward(d_bi, dHn, np.zeros((B, S, 4, D)), wn[:, 0:4], wn[:, 8:].reshape(B, 4, 4))
        return torch.tensor(dH + gx.reshape(B, 1, 4, D) / S)


def _unfused_case(monkeypatch):
    from mhc import _kernels, module
    from mhc._torch_baseline import sinkhorn_knopp_torch

    for name in ("branch_input", "mix_backward", "mix_dh"):
        monkeypatch.setattr(_layer, name, getattr(_UnfusedLaunchers, name))
    for name in ("add_forward", "add_backward"):
        monkeypatch.setattr(_layer, name, getattr(_OracleLaunchers, name))
    monkeypatch.setattr(_kernels, "mean_pool", _UnfusedLaunchers.mean_pool)
    monkeypatch.setattr(module, "sinkhorn_knopp", sinkhorn_knopp_torch)
    # node A hands the kernels fp32 weights; float64 here keeps the check at rounding level
    monkeypatch.setattr(_layer, "_f32", lambda t: t.contiguous())
    g = np.random.default_rng(5)
    B, S, D = 2, 3, 4
    hc = mhc.HyperConnection(D, dynamic=True, use_fused_weights=False).double()
    with torch.no_grad():
        for prm in hc.parameters():
            prm.copy_(torch.tensor(g.standard_normal(tuple(prm.shape)) * 0.5))
    p = {n.replace(".weight", ""): prm.detach().numpy().copy() for n, prm in hc.named_parameters()}
    arrays = [g.standard_normal(s) for s in ((B, S, 4, D), (B, S, D), (B, S, 4, D), (B, S, D))]
    return hc, p, arrays


def _unfused_grads_close(hc, H, g):
    g = {k.replace(".weight", ""): v for k, v in g.items()}
    assert np.abs(H.grad.numpy() - g["H"]).max() < 1e-12
    for n, prm in hc.named_parameters():
        k = n.replace(".weight", "")
        assert np.abs(prm.grad.numpy() - g[k].reshape(prm.shape)).max() < 1e-12, n


def test_unfused_layer_writes_dh_in_the_pool_node(monkeypatch):
    """Unfused dynamic layer, closure called twice: node A hands dH_new, d_branch_input and w to
    the sequence-mean node, which adds grad_x / S itself; dH and every parameter gradient equal
    the oracle's (the sum over the two closure calls)."""
    hc, p, (H_np, bo_np, dHn_np, dbi_np) = _unfused_case(monkeypatch)
    H = torch.tensor(H_np, requires_grad=True)
    bi, add = hc(H)
    Hn1 = add(torch.tensor(bo_np))
    Hn2 = add(torch.tensor(2 * bo_np))
    torch.autograd.backward([Hn1, Hn2, bi], [torch.tensor(dHn_np), torch.tensor(0.5 * dHn_np), torch.tensor(dbi_np)])
    _, _, c1 = O.layer_forward(p, H_np, bo_np, dynamic=True, fused=False, iters=hc.sinkhorn_iters, eps=hc.eps)
    _, _, c2 = O.layer_forward(p, H_np, 2 * bo_np, dynamic=True, fused=False, iters=hc.sinkhorn_iters, eps=hc.eps)
    g1 = O.layer_backward(p, c1, dHn_np, dbi_np)
    g2 = O.layer_backward(p, c2, 0.5 * dHn_np, np.zeros_like(dbi_np))
    _unfused_grads_close(hc, H, {k: g1[k] + g2[k] for k in g1})


def test_unfused_partial_backward_then_branch_input(monkeypatch):
    """autograd.grad(H_new, branch_output) runs only the closure; bi.backward() afterwards gives
    the branch_input-only gradients, with grad_x / S still folded into dH by the pool node."""
    hc, p, (H_np, bo_np, dHn_np, dbi_np) = _unfused_case(monkeypatch)
    H = torch.tensor(H_np, requires_grad=True)
    bo = torch.tensor(bo_np, requires_grad=True)
    bi, add = hc(H)
    Hn = add(bo)
    (d_bo,) = torch.autograd.grad(Hn, bo, torch.tensor(dHn_np), retain_graph=True)
    _, _, cache = O.layer_forward(p, H_np, bo_np, dynamic=True, fused=False, iters=hc.sinkhorn_iters, eps=hc.eps)
    assert np.abs(d_bo.numpy() - O.layer_backward(p, cache, dHn_np, dbi_np)["bo"]).max() < 1e-12
    bi.backward(torch.tensor(dbi_np))
    _unfused_grads_close(hc, H, O.layer_backward(p, cache, np.zeros_like(dHn_np), dbi_np))


def test_unfused_parameters_only_and_h_without_grad(monkeypatch):
    """Gradients of the parameters alone (the pool node's backward is not needed and does not
    run), and a forward on an H that does not require grad (no pool node is recorded)."""
    hc, p, (H_np, bo_np, dHn_np, dbi_np) = _unfused_case(monkeypatch)
    _, _, cache = O.layer_forward(p, H_np, bo_np, dynamic=True, fused=False, iters=hc.sinkhorn_iters, eps=hc.eps)
    full = {k.replace(".weight", ""): v for k, v in O.layer_backward(p, cache, dHn_np, dbi_np).items()}
    H = torch.tensor(H_np, requires_grad=True)
    bi, add = hc(H)
    Hn = add(torch.tensor(bo_np))
    params = list(hc.named_parameters())
    gs = torch.autograd.grad([Hn, bi], [prm for _, prm in params], [torch.tensor(dHn_np), torch.tensor(dbi_np)])
    for (n, prm), gv in zip(params, gs):
        k = n.replace(".weight", "")
        assert np.abs(gv.numpy() - full[k].reshape(prm.shape)).max() < 1e-12, n
    assert H.grad is None
    bi, add = hc(torch.tensor(H_np))
    torch.autograd.backward([add(torch.tensor(bo_np)), bi], [torch.tensor(dHn_np), torch.tensor(dbi_np)])
    for n, prm in hc.named_parameters():
        k = n.replace(".weight", "")
        assert np.abs(prm.grad.numpy() - full[k].reshape(prm.shape)).max() < 1e-12, n


def _static_case(monkeypatch):
    for name in ("static_forward", "static_backward", "add_forward", "add_backward"):
        monkeypatch.setattr(_layer, name, getattr(_OracleLaunchers, name))
    g = np.random.default_rng(3)
    B, S, D = 2, 3, 4
    hc = mhc.HyperConnection(D, dynamic=False).double()
    p = {"H_pre_base": g.standard_normal(4), "H_post_base": g.standard_normal(4),
         "H_res_base": g.standard_normal((4, 4))}
    with torch.no_grad():
        for n, prm in hc.named_parameters():
            prm.copy_(torch.tensor(p[n]))
    arrays = [g.standard_normal(s) for s in ((B, S, 4, D), (B, S, D), (B, S, 4, D), (B, S, D))]
    return hc, p, arrays


def _grads_close(hc, H, g, keys=("H_pre_base", "H_post_base", "H_res_base")):
    assert np.abs(H.grad.numpy() - g["H"]).max() < 1e-12
    for n, prm in hc.named_parameters():
        assert np.abs(prm.grad.numpy() - g[n].reshape(prm.shape)).max() < 1e-12, n


def test_partial_backward_leaves_no_closure_gradient_behind(monkeypatch):
    """A backward call that reaches the closure but not node A (here autograd.grad w.r.t.
    branch_output only) must not leak into a later backward: H.grad and the parameter grads
    of bi.backward() afterwards are the branch_input-only gradients."""
    hc, p, (H_np, bo_np, dHn_np, dbi_np) = _static_case(monkeypatch)
    H = torch.tensor(H_np, requires_grad=True)
    bo = torch.tensor(bo_np, requires_grad=True)
    bi, add = hc(H)
    Hn = add(bo)
    (d_bo,) = torch.autograd.grad(Hn, bo, torch.tensor(dHn_np), retain_graph=True)
    _, _, cache = O.layer_forward(p, H_np, bo_np, dynamic=False)
    full = O.layer_backward(p, cache, dHn_np, dbi_np)
    assert np.abs(d_bo.numpy() - full["bo"]).max() < 1e-12
    bi.backward(torch.tensor(dbi_np))
    _grads_close(hc, H, O.layer_backward(p, cache, np.zeros_like(dHn_np), dbi_np))


def test_closure_gradients_reach_node_a_and_sum_over_calls(monkeypatch):
    """Full backward through bi and two closure calls: the engine sums the two link / w
    gradients, and node A sees their sum (the closure is linear in dH_new)."""
    hc, p, (H_np, bo_np, dHn_np, dbi_np) = _static_case(monkeypatch)
    H = torch.tensor(H_np, requires_grad=True)
    bi, add = hc(H)
    Hn1 = add(torch.tensor(bo_np))
    Hn2 = add(torch.tensor(2 * bo_np))
    torch.autograd.backward([Hn1, Hn2, bi], [torch.tensor(dHn_np), torch.tensor(0.5 * dHn_np), torch.tensor(dbi_np)])
    _, _, c1 = O.layer_forward(p, H_np, bo_np, dynamic=False)
    _, _, c2 = O.layer_forward(p, H_np, 2 * bo_np, dynamic=False)
    g1 = O.layer_backward(p, c1, dHn_np, dbi_np)
    g2 = O.layer_backward(p, c2, 0.5 * dHn_np, np.zeros_like(dbi_np))
    _grads_close(hc, H, {k: g1[k] + g2[k] for k in g1})


def test_closure_rejects_in_place_change_of_H(monkeypatch):
    """The closure recomputes H_res @ H from H; an in-place change of H after forward would
    silently change H_new (the reference's closure holds H_residual), so it raises."""
    hc, p, (H_np, bo_np, _, _) = _static_case(monkeypatch)
    H = torch.tensor(H_np)
    bi, add = hc(H)
    with torch.no_grad():
        H.mul_(2.0)
    with pytest.raises(RuntimeError, match="modified in place"):
        add(torch.tensor(bo_np))
    bi, add = hc(H)
    _, want, _ = O.layer_forward(p, 2 * H_np, bo_np, dynamic=False)
    assert np.abs(add(torch.tensor(bo_np)).detach().numpy() - want).max() < 1e-12
    # a strided H is copied once in forward: changing the original afterwards is harmless
    Hs = torch.tensor(H_np).transpose(1, 3).contiguous().transpose(1, 3)
    assert not Hs.is_contiguous()
    bi, add = hc(Hs)
    with torch.no_grad():
        Hs.zero_()
    _, want, _ = O.layer_forward(p, H_np, bo_np, dynamic=False)
    assert np.abs(add(torch.tensor(bo_np)).detach().numpy() - want).max() < 1e-12


def test_bench_cpu_baseline_fields():
    """bench.py's cpu_baseline leg (the reference's torch layer restated, on the host cores) reports
    the contract's fields plus the host and torch version it ran on (here on a short sequence)."""
    import importlib.util
    import os

    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "bench.py")
    spec = importlib.util.spec_from_file_location("mhc_bench", path)
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    for w in ("config3", "config5"):
        r = bench._cpu_leg(dict(bench.WORKLOADS[w]), reps=1, seq=8)
        assert set(r) >= {"value", "unit", "cores", "kind", "sample", "host_cpus", "host_cpu_model",
                          "torch_version", "fwd_only_tokens_per_s", "runs_s"}
        assert r["value"] > 0 and r["unit"] == "tokens/s" and r["kind"] == "port"
        assert r["cores"] == torch.get_num_threads() and r["host_cpus"] == os.cpu_count()
        assert r["torch_version"] == torch.__version__ and "S=8 " in r["sample"]
