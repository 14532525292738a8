"""A hyper-connection stack trained on the HIP path follows the same trajectory as the same stack
built from the reference's pure-PyTorch ``HyperConnectionTorch`` (the public baseline a user would
swap out).

The model: embeddings expanded to four streams, three blocks of ``HyperConnection`` around an
MLP branch, the streams collapsed by their mean, a linear head and an MSE loss.  Both stacks start
from the same state dict and take the same SGD-with-momentum steps on one batch, in fp32
on the GPU (torch ops for the baseline).  SGD keeps the parameter updates linear in the gradients,
so fp32 rounding differences stay of their own size instead of being rescaled per element."""

import pytest
import torch

from helpers import rel_err, to_np

pytestmark = pytest.mark.gpu

DEV = "cuda"


class Stack(torch.nn.Module):
    def __init__(self, hc_cls, D, layers, dynamic, fused, expand, collapse):
        super().__init__()
        self.hcs = torch.nn.ModuleList(hc_cls(D, layer_idx=i, dynamic=dynamic, use_fused_weights=fused)
                                       for i in range(layers))
        self.branches = torch.nn.ModuleList(
            torch.nn.Sequential(torch.nn.Linear(D, 2 * D), torch.nn.GELU(), torch.nn.Linear(2 * D, D))
            for _ in range(layers))
        self.head = torch.nn.Linear(D, D)
        self.expand, self.collapse = expand, collapse

    def forward(self, x):
        H = self.expand(x)
        for hc, branch in zip(self.hcs, self.branches):
            bi, add = hc(H)
            H = add(branch(bi))
        return self.head(self.collapse(H))


@pytest.mark.parametrize("dynamic,fused", [(True, True), (False, True), (True, False)])
def test_stack_trains_like_the_torch_baseline(dynamic, fused):
    import mhc
    from mhc.streams import collapse_streams, expand_streams

    B, S, D, layers, steps = 2, 32, 64, 3, 5
    torch.manual_seed(0)
    hip = Stack(mhc.HyperConnection, D, layers, dynamic, fused, expand_streams,
                lambda H: collapse_streams(H, reduction="mean")).to(DEV)
    ref = Stack(mhc.HyperConnectionTorch, D, layers, dynamic, fused,
                lambda x: x.unsqueeze(2).expand(-1, -1, 4, -1), lambda H: H.mean(dim=2)).to(DEV)
    with torch.no_grad():
        # non-zero dynamic-weight parameters, so that every weight path carries gradient
        for hc in hip.hcs:
            if dynamic and fused:
                hc.phi.normal_(0.0, 0.05)
            elif dynamic:
                for lin in (hc.W_pre, hc.W_post, hc.W_res):
                    lin.weight.normal_(0.0, 0.05)
    ref.load_state_dict(hip.state_dict())
    opts = [torch.optim.SGD(m.parameters(), lr=0.05, momentum=0.9) for m in (hip, ref)]
    g = torch.Generator(device=DEV).manual_seed(1)
    x = torch.randn((B, S, D), generator=g, device=DEV)  # one batch, fitted for a few steps
    y = torch.randn((B, S, D), generator=g, device=DEV)
    losses = []
    for _ in range(steps):
        step = []
        for m, opt in zip((hip, ref), opts):
            opt.zero_grad(set_to_none=True)
            loss = torch.nn.functional.mse_loss(m(x), y)
            loss.backward()
            opt.step()
            step.append(loss.item())
        losses.append(step)
    print("losses (hip, torch):", [(round(a, 6), round(b, 6)) for a, b in losses], flush=True)
    for a, b in losses:
        assert abs(a - b) <= 1e-5 * abs(b), losses
    assert losses[-1][0] < losses[0][0]  # it trains
    ref_params = dict(ref.named_parameters())
    worst = max(rel_err(to_np(p), to_np(ref_params[n])) for n, p in hip.named_parameters())
    print(f"worst parameter error after {steps} steps: {worst:.2e}", flush=True)
    assert worst < 1e-4
