"""Host logic that needs no GPU: module construction / parameters / init
(reference src/mhc/module.py:37-101,191-224), the public API surface, the
pure-PyTorch baselines on CPU, and the node-B -> node-A gradient stash."""

import numpy as np
import torch

import mhc
from mhc import _layer


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


def test_stash_sums_repeated_closure_gradients():
    s = _layer._Stash()
    assert s.take() == (None, None)
    a, b = torch.ones(2, 3), torch.full((2, 4), 2.0)
    s.put(a, b)
    s.put(a * 3, b * 5)
    dh, dp = s.take()
    assert torch.equal(dh, torch.full((2, 3), 4.0)) and torch.equal(dp, torch.full((2, 4), 12.0))
    assert s.take() == (None, None)


def test_bench_cpu_baseline_fields():
    """bench.py's cpu_baseline leg (the reference's torch layer restated, on the host cores) reports
    the contract's fields plus the host it ran on, on a short sample."""
    import importlib.util
    import os

    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "bench.py")
    spec = importlib.util.spec_from_file_location("mhc_bench", path)
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    r = bench._cpu_leg(dict(bench.WORKLOADS["config5"]), 0.2)
    assert set(r) >= {"value", "unit", "cores", "kind", "sample", "host_cpus", "host_cpu_model"}
    assert r["value"] > 0 and r["unit"] == "tokens/s" and r["kind"] == "port"
    assert r["cores"] == torch.get_num_threads() and r["host_cpus"] == os.cpu_count()
