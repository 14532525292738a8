"""HIP-graph capture of the HyperConnection layer, forward and backward.

The layer path makes no host synchronisation (the alphas stay on the
device), allocates only through torch's caching allocator and clears memory
with kernels, never hipMemsetAsync, so a whole training step of the layer can
be captured with torch.cuda.graph and replayed.  Each replay must reproduce
the eager step bit for bit (every kernel is deterministic): checked on several
replays in a row, with eager work and synchronisations between them, and after
new values are copied into the captured input tensors.  The replayed outputs and
gradients are also checked against the float64 oracle layer on the same inputs
(fp32: 1e-5 forward, 1e-4 gradients; bf16: 2e-2).
"""

import numpy as np
import pytest
import torch

from helpers import rel_err, to_np
from oracle import mhc_oracle as O

pytestmark = pytest.mark.gpu


def _check_oracle(hc, H, bo, dHn, dbi, got, dtype):
    """Replayed outputs and gradients against the float64 oracle layer."""
    p = {n.replace(".weight", ""): to_np(v) for n, v in hc.named_parameters()}
    fused = hc.use_fused_weights or not hc.dynamic
    obi, oHn, cache = O.layer_forward(p, to_np(H), to_np(bo), hc.dynamic, fused, hc.sinkhorn_iters, hc.eps)
    og = O.layer_backward(p, cache, to_np(dHn), to_np(dbi))
    ftol, gtol = (1e-5, 1e-4) if dtype == torch.float32 else (2e-2, 2e-2)
    assert rel_err(to_np(got["bi"]), obi) < ftol and rel_err(to_np(got["H_new"]), oHn) < ftol
    assert rel_err(to_np(got["dH"]), og["H"]) < gtol and rel_err(to_np(got["dbo"]), og["bo"]) < gtol
    for n, _ in hc.named_parameters():
        want = og[n]
        err = rel_err(to_np(got["d" + n]).reshape(np.shape(want)), want)
        print(f"replay d{n}: {err:.2e}", flush=True)
        assert err < 1e-4, n


def _setup(dynamic, fused=True, seed=0, dtype=torch.bfloat16, shape=(2, 64, 256)):
    import mhc

    B, S, D = shape
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    hc = mhc.HyperConnection(D, dynamic=dynamic, use_fused_weights=fused).cuda()
    with torch.no_grad():
        if dynamic and fused:
            hc.phi.copy_(torch.randn(hc.phi.shape, generator=g, device="cuda") * 0.02)
        if not dynamic:
            hc.H_res_base.copy_(torch.randn((4, 4), generator=g, device="cuda"))
    mk = lambda *shape: torch.randn(shape, generator=g, device="cuda").to(dtype)  # noqa: E731
    H = mk(B, S, 4, D).requires_grad_(True)
    bo = mk(B, S, D).requires_grad_(True)
    return hc, H, bo, mk(B, S, 4, D), mk(B, S, D), mk


def _step(hc, H, bo, dHn, dbi):
    H.grad = None
    bo.grad = None
    for p in hc.parameters():
        p.grad = None
    bi, add = hc(H)
    H_new = add(bo)
    torch.autograd.backward([H_new, bi], [dHn, dbi])
    return bi, H_new


def _snapshot(hc, H, bo, bi, H_new):
    out = {"bi": bi.detach().clone(), "H_new": H_new.detach().clone(), "dH": H.grad.clone(), "dbo": bo.grad.clone()}
    out.update({"d" + n: p.grad.clone() for n, p in hc.named_parameters()})
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("dynamic,fused", [(True, True), (False, True), (True, False)])
def test_layer_step_graph_replays_match_eager(dynamic, fused, dtype):
    _graph_replays_match_eager(*_setup(dynamic, fused, dtype=dtype), dtype)


@pytest.mark.parametrize("shape", [(600, 1, 128), (130, 2, 4096)])
def test_many_sequences_graph_replays_match_eager(shape):
    """Many short sequences, dynamic fused weights: the bulk-batch paths (the projection and the
    weights backward on the MFMA kernels; at S = 1 both read H's rows, with no pooled rows kept)."""
    _graph_replays_match_eager(*_setup(True, True, dtype=torch.bfloat16, shape=shape), torch.bfloat16)


def _graph_replays_match_eager(hc, H, bo, dHn, dbi, mk, dtype):
    ref = _snapshot(hc, H, bo, *_step(hc, H, bo, dHn, dbi))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            _step(hc, H, bo, dHn, dbi)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    H.grad = None
    bo.grad = None
    for p in hc.parameters():
        p.grad = None
    with torch.cuda.graph(graph):
        bi_g, H_new_g = _step(hc, H, bo, dHn, dbi)

    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        got = _snapshot(hc, H, bo, bi_g, H_new_g)
        for k, v in ref.items():
            assert torch.equal(got[k], v), (i, k)
        if i == 0:
            _check_oracle(hc, H, bo, dHn, dbi, got, dtype)
        # unrelated eager work between replays
        x = mk(1024, 1024).float()
        (x @ x).sum().item()

    # new input values in the captured tensors: replay == eager on the new values
    with torch.no_grad():
        H.copy_(mk(*H.shape))
        bo.copy_(mk(*bo.shape))
        dHn.copy_(mk(*dHn.shape))
    graph.replay()
    torch.cuda.synchronize()
    got = _snapshot(hc, H, bo, bi_g, H_new_g)
    want = _snapshot(hc, H, bo, *_step(hc, H, bo, dHn, dbi))
    for k, v in want.items():
        assert torch.equal(got[k], v), ("new inputs", k)
    _check_oracle(hc, H, bo, dHn, dbi, got, dtype)
