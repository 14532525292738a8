"""HyperConnection forward + backward at the full BASELINE.json sizes (configs
3, 4 and 5), where the float64 oracle cannot run on the whole layer.

What is checked, per config:
* the dynamic (or static) weights: the oracle computes them from the sequence
  mean of H (taken by torch in float64 on the GPU, a [B, 4D] result) and the
  module parameters;
* branch_input, H_new, dH and d branch_output: against torch fp32 arithmetic
  on the GPU with the oracle's weights (normwise relative error <= 2e-2, the
  bf16/fp16 output tolerance);
* every parameter gradient: the oracle's weight backward fed float64
  reductions of the upstream gradients, taken on the GPU (dH_pre = sum d_bi * H[n],
  dH_res = sum dH_new[n] * H[m], dH_post = sum dH_new[n] * bo over all S * D
  terms) and the float64 sequence mean, <= 1e-4 (the fp32-gradient tolerance);
* branch_input, H_new, d branch_output and dH once more, against the float64
  value of each expression from the layer's own fp32 weights, rounded once to
  the bf16 / fp16 output: within one unit in the last place, and bit-identical
  but for a small fraction (test_gpu_rounding.check_layer_rounding).
These exercise the kernels' index arithmetic at the real shapes (up to 2^28
elements per tensor) and the split-S / split-K reduction plans.
"""

import numpy as np
import pytest
import torch

from helpers import rel_err, to_np
from oracle import mhc_oracle as O
from test_gpu_rounding import _red, _red44, check_layer_rounding

pytestmark = pytest.mark.gpu

CONFIGS = {
    "config3": dict(B=4, S=4096, D=4096, dtype=torch.bfloat16, dynamic=True),
    "config4": dict(B=1, S=8192, D=7168, dtype=torch.bfloat16, dynamic=True),
    "config5": dict(B=16, S=2048, D=2048, dtype=torch.float16, dynamic=False),
}


@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_full_size_layer(name):
    import mhc

    c = CONFIGS[name]
    B, S, D, dt = c["B"], c["S"], c["D"], c["dtype"]
    print(f"full-size {name}: B={B} S={S} D={D} {dt}", flush=True)
    dev = "cuda"
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    hc = mhc.HyperConnection(D, dynamic=c["dynamic"]).to(dev)
    H = torch.randn((B, S, 4, D), generator=g, device=dev).to(dt)
    with torch.no_grad():
        if c["dynamic"]:
            hc.phi.copy_(torch.randn((24, 4 * D), generator=g, device=dev).T * 0.02)
        else:
            hc.H_res_base.copy_(torch.randn((4, 4), generator=g, device=dev))
    bo = torch.randn((B, S, D), generator=g, device=dev).to(dt)
    dHn = torch.randn((B, S, 4, D), generator=g, device=dev).to(dt)
    dbi = torch.randn((B, S, D), generator=g, device=dev).to(dt)
    Hl = H.clone().requires_grad_(True)
    bol = bo.clone().requires_grad_(True)
    bi, add = hc(Hl)
    H_new = add(bol)
    torch.autograd.backward([H_new, bi], [dHn, dbi])
    torch.cuda.synchronize()

    p = {n: to_np(v) for n, v in hc.named_parameters()}
    Hf = H.float()
    if c["dynamic"]:
        x = to_np(H.double().mean(dim=1).reshape(B, 4 * D))
        bias = np.concatenate([p["H_pre_base"], p["H_post_base"], p["H_res_base"].reshape(16)])
        al = [float(p[k][0]) for k in ("alpha_pre", "alpha_post", "alpha_res")]
        H_pre, H_post, H_res = O.dynamic_weights(x, p["phi"], bias, *al, 20, 1e-6)
    else:
        H_post, H_pre, H_res = O.static_weights(p["H_pre_base"], p["H_post_base"], p["H_res_base"], B, 20)
    wp = torch.tensor(H_pre, dtype=torch.float32, device=dev)
    wq = torch.tensor(H_post, dtype=torch.float32, device=dev)
    wr = torch.tensor(H_res, dtype=torch.float32, device=dev)

    # forward
    bi_ref = (wp[:, None, :, None] * Hf).sum(dim=2)
    assert rel_err(to_np(bi), to_np(bi_ref)) < 2e-2
    del bi_ref
    hn_ref = torch.empty_like(Hf)
    for n in range(4):
        hn_ref[:, :, n] = (wr[:, n, None, :, None] * Hf).sum(dim=2) + wq[:, n, None, None] * bo.float()
    assert rel_err(to_np(H_new), to_np(hn_ref)) < 2e-2
    del hn_ref

    # upstream reductions in float64 on the GPU, weight backward in the oracle
    dbf, dnf = dbi.float(), dHn.float()
    H64 = H.double()
    dpre = to_np(_red(dbi.double(), H64))
    dres = to_np(_red44(dHn.double(), H64))
    del H64
    dpost = to_np(_red(bo.double(), dHn.double()))
    if c["dynamic"]:
        gx, gphi, gbias, ga = O.dynamic_weights_backward(x, p["phi"], bias, *al, dpre, dpost, dres, 20, 1e-6)
        ref = {"phi": gphi, "H_pre_base": gbias[0:4], "H_post_base": gbias[4:8],
               "H_res_base": gbias[8:24].reshape(4, 4), "alpha_pre": np.array([ga[0]]),
               "alpha_post": np.array([ga[1]]), "alpha_res": np.array([ga[2]])}
    else:
        gq, gp, gr = O.static_weights_backward(p["H_pre_base"], p["H_post_base"], p["H_res_base"], dpost, dpre,
                                               dres, 20)
        ref = {"H_pre_base": gq, "H_post_base": gp, "H_res_base": gr}
        gx = None
    perr = {n: rel_err(to_np(prm.grad).reshape(ref[n].shape), ref[n]) for n, prm in hc.named_parameters()}
    print(f"full-size {name} parameter gradients:", {n: f"{e:.2e}" for n, e in perr.items()}, flush=True)
    for n, e in perr.items():
        assert e < 1e-4, (n, perr)

    # dH = H_pre d_bi + H_res^T dH_new (+ grad_x / S) and d_bo = sum_n H_post[n] dH_new[n]
    dH_ref = wp[:, None, :, None] * dbf[:, :, None, :]
    for m in range(4):
        dH_ref[:, :, m] += sum(wr[:, n, m, None, None] * dnf[:, :, n] for n in range(4))
    if gx is not None:
        dH_ref += torch.tensor(gx, dtype=torch.float32, device=dev).reshape(B, 1, 4, D) / S
    assert rel_err(to_np(Hl.grad), to_np(dH_ref)) < 2e-2
    del dH_ref
    dbo_ref = (wq[:, None, :, None] * dnf).sum(dim=2)
    assert rel_err(to_np(bol.grad), to_np(dbo_ref)) < 2e-2
    del dbo_ref, Hl, bol, bi, H_new, dbf, dnf, Hf
    torch.cuda.empty_cache()
    check_layer_rounding("dynamic" if c["dynamic"] else "static", hc, H, bo, dHn, dbi)
