"""The reference's own test suite (reference tests/test_mhc.py), case by case, on this build.

Each case keeps the reference test's seed, shapes, checks and tolerances; the class and method
names are the reference's, so that a run of this file reads as that suite passing on the
MI355X.  The comparison math is restated here in plain fp32 torch (broadcast products and sums,
no einsum), as the reference's tests restate theirs.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def sinkhorn_plain(M, iters=20, eps=1e-8):
    """|M| + eps, then `iters` rounds of row and column normalisation (test_mhc.py:13-19)."""
    P = M.abs() + eps
    for _ in range(iters):
        P = P / (P.sum(-1, keepdim=True) + eps)
        P = P / (P.sum(-2, keepdim=True) + eps)
    return P


def mix_plain(H, H_pre, H_res):
    """branch_input[b,s,:] = sum_n H_pre[b,n] H[b,s,n,:]; H_residual[b,s,n,:] = sum_m
    H_res[b,n,m] H[b,s,m,:]."""
    branch = (H_pre[:, None, :, None] * H).sum(2)
    residual = (H_res[:, None, :, :, None] * H[:, :, None, :, :]).sum(3)
    return branch, residual


def add_plain(H_residual, branch_out, H_post):
    return H_residual + branch_out[:, :, None, :] * H_post[:, None, :, None]


class TestSinkhornKnopp:
    """test_mhc.py:22-64."""

    def test_forward_correctness(self):
        from mhc import sinkhorn_knopp

        torch.manual_seed(42)
        M = torch.randn(4, 4, 4, device=DEV)
        assert (sinkhorn_plain(M.clone()) - sinkhorn_knopp(M.clone())).abs().max() < 1e-5

    def test_doubly_stochastic(self):
        from mhc import sinkhorn_knopp

        torch.manual_seed(42)
        P = sinkhorn_knopp(torch.randn(8, 4, 4, device=DEV))
        ones = torch.ones(8, 4, device=DEV)
        assert torch.allclose(P.sum(-1), ones, atol=1e-4)
        assert torch.allclose(P.sum(-2), ones, atol=1e-4)

    def test_backward(self):
        from mhc import sinkhorn_knopp

        torch.manual_seed(42)
        M = torch.randn(4, 4, 4, device=DEV, requires_grad=True)
        M_hip = M.detach().clone().requires_grad_(True)
        sinkhorn_plain(M).sum().backward()
        sinkhorn_knopp(M_hip).sum().backward()
        assert (M.grad - M_hip.grad).abs().max() < 1e-4


class TestStreamMix:
    """test_mhc.py:67-114."""

    def test_forward_correctness(self):
        from mhc import fused_stream_mix

        torch.manual_seed(42)
        B, S, D = 2, 64, 256
        H = torch.randn(B, S, 4, D, device=DEV)
        H_pre = torch.softmax(torch.randn(B, 4, device=DEV), dim=-1)
        H_res = sinkhorn_plain(torch.randn(B, 4, 4, device=DEV))
        want_bi, want_res = mix_plain(H, H_pre, H_res)
        bi, res = fused_stream_mix(H, H_pre, H_res)
        assert (want_bi - bi).abs().max() < 1e-4
        assert (want_res - res).abs().max() < 1e-4

    def test_backward(self):
        from mhc import fused_stream_mix

        torch.manual_seed(42)
        B, S, D = 2, 32, 128
        H = torch.randn(B, S, 4, D, device=DEV, requires_grad=True)
        H_pre = torch.softmax(torch.randn(B, 4, device=DEV), dim=-1).requires_grad_(True)
        H_res = sinkhorn_plain(torch.randn(B, 4, 4, device=DEV)).detach().requires_grad_(True)
        hip = [t.detach().clone().requires_grad_(True) for t in (H, H_pre, H_res)]
        sum(t.sum() for t in mix_plain(H, H_pre, H_res)).backward()
        sum(t.sum() for t in fused_stream_mix(*hip)).backward()
        assert (H.grad - hip[0].grad).abs().max() < 1e-3


class TestAddResidual:
    """test_mhc.py:117-161."""

    def test_forward_correctness(self):
        from mhc import fused_add_residual

        torch.manual_seed(42)
        B, S, D = 2, 64, 256
        H_residual = torch.randn(B, S, 4, D, device=DEV)
        branch_out = torch.randn(B, S, D, device=DEV)
        H_post = torch.sigmoid(torch.randn(B, 4, device=DEV))
        got = fused_add_residual(H_residual, branch_out, H_post)
        assert (add_plain(H_residual, branch_out, H_post) - got).abs().max() < 1e-4

    def test_backward(self):
        from mhc import fused_add_residual

        torch.manual_seed(42)
        B, S, D = 2, 32, 128
        H_res = torch.randn(B, S, 4, D, device=DEV, requires_grad=True)
        branch = torch.randn(B, S, D, device=DEV, requires_grad=True)
        H_post = torch.sigmoid(torch.randn(B, 4, device=DEV)).requires_grad_(True)
        hip = [t.detach().clone().requires_grad_(True) for t in (H_res, branch, H_post)]
        add_plain(H_res, branch, H_post).sum().backward()
        fused_add_residual(*hip).sum().backward()
        assert (H_res.grad - hip[0].grad).abs().max() < 1e-3


class TestHyperConnection:
    """test_mhc.py:164-216."""

    def test_forward_shape(self):
        from mhc import HyperConnection

        hc = HyperConnection(dim=256, dynamic=True).to(DEV)
        branch_input, add_residual = hc(torch.randn(2, 64, 4, 256, device=DEV))
        assert branch_input.shape == (2, 64, 256)
        assert add_residual(torch.randn(2, 64, 256, device=DEV)).shape == (2, 64, 4, 256)

    def test_training(self):
        from mhc import HyperConnection

        torch.manual_seed(42)
        hc = HyperConnection(dim=128, dynamic=True).to(DEV)
        layer = torch.nn.Linear(128, 128, device=DEV)
        opt = torch.optim.Adam(list(hc.parameters()) + list(layer.parameters()))
        before = {n: p.detach().clone() for n, p in hc.named_parameters()}
        for _ in range(3):
            opt.zero_grad()
            H = torch.randn(2, 32, 4, 128, device=DEV, requires_grad=True)
            branch_input, add_residual = hc(H)
            add_residual(layer(branch_input)).sum().backward()
            opt.step()
        changed = [n for n, p in hc.named_parameters() if not torch.allclose(p, before[n])]
        assert changed, "parameters should update during training"

    def test_static_mode(self):
        from mhc import HyperConnection

        hc = HyperConnection(dim=128, dynamic=False).to(DEV)
        branch_input, _ = hc(torch.randn(2, 32, 4, 128, device=DEV))
        assert branch_input.shape == (2, 32, 128)
