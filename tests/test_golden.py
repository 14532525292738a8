"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from the float64 oracle).

CPU: the oracle still reproduces every fixture (a regression pin on the oracle,
which tests/test_oracle.py pins against closed forms, finite differences and
torch autograd).
GPU: the HIP path, fed the fixtures' inputs in fp32, matches the fixtures'
outputs and gradients within the fp32 tolerances (normwise relative error:
forward 1e-5, gradients 1e-4).
"""

import glob
import os

import numpy as np
import pytest
import torch

from helpers import rel_err, to_np
from oracle import mhc_oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FWD, GRAD = 1e-5, 1e-4


def load(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def layer_params(z):
    return {k[2:]: v for k, v in z.items() if k.startswith("p_")}


def layer_flags(name):
    return {"layer_dynamic_init.npz": (True, True), "layer_dynamic.npz": (True, True),
            "layer_static.npz": (False, True), "layer_unfused.npz": (True, False)}[name]


LAYERS = ["layer_dynamic_init.npz", "layer_dynamic.npz", "layer_static.npz", "layer_unfused.npz"]


def test_fixture_set_present():
    names = sorted(os.path.basename(p) for p in glob.glob(os.path.join(GOLDEN, "*.npz")))
    assert names == sorted(["sinkhorn_20.npz", "sinkhorn_7.npz", "dynamic_weights.npz", "stream_ops.npz"] + LAYERS)


@pytest.mark.parametrize("name", ["sinkhorn_20.npz", "sinkhorn_7.npz"])
def test_oracle_reproduces_sinkhorn(name):
    z = load(name)
    it, eps = int(z["iters"]), float(z["eps"])
    assert np.allclose(O.sinkhorn(z["M"], it, eps), z["P"], rtol=0, atol=1e-13)
    assert np.allclose(O.sinkhorn_backward(z["M"], z["dP"], it, eps), z["dM"], rtol=0, atol=1e-12)


def test_oracle_reproduces_dynamic_weights():
    z = load("dynamic_weights.npz")
    out = O.dynamic_weights(z["x"], z["phi"], z["bias"], *z["alphas"], 20, 1e-6)
    for k, v in zip(("H_pre", "H_post", "H_res"), out):
        assert np.allclose(v, z[k], rtol=0, atol=1e-13), k
    gx, gphi, gbias, ga = O.dynamic_weights_backward(z["x"], z["phi"], z["bias"], *z["alphas"], z["gH_pre"],
                                                     z["gH_post"], z["gH_res"], 20, 1e-6)
    for v, k in ((gx, "gx"), (gphi, "gphi"), (gbias, "gbias"), (np.array(ga), "galpha")):
        assert np.allclose(v, z[k], rtol=0, atol=1e-12), k


def test_oracle_reproduces_stream_ops():
    z = load("stream_ops.npz")
    bi, hr = O.stream_mix(z["H"], z["H_pre"], z["H_res"])
    assert np.allclose(bi, z["bi"], atol=1e-13) and np.allclose(hr, z["hr"], atol=1e-13)
    dH, dpre, dres = O.stream_mix_backward(z["d_bi"], z["d_hr"], z["H"], z["H_pre"], z["H_res"])
    for v, k in ((dH, "dH"), (dpre, "dpre"), (dres, "dres")):
        assert np.allclose(v, z[k], atol=1e-12), k
    assert np.allclose(O.add_residual(z["hr"], z["bo"], z["H_post"]), z["H_new"], atol=1e-13)
    _, d_bo, dpost = O.add_residual_backward(z["dHn"], z["bo"], z["H_post"])
    assert np.allclose(d_bo, z["d_bo"], atol=1e-12) and np.allclose(dpost, z["dpost"], atol=1e-12)


@pytest.mark.parametrize("name", LAYERS)
def test_oracle_reproduces_layer(name):
    z = load(name)
    dynamic, fused = layer_flags(name)
    p = layer_params(z)
    bi, H_new, cache = O.layer_forward(p, z["H"], z["bo"], dynamic, fused, 20, 1e-6)
    assert np.allclose(bi, z["bi"], atol=1e-13) and np.allclose(H_new, z["H_new"], atol=1e-13)
    g = O.layer_backward(p, cache, z["dHn"], z["dbi"])
    for k, v in g.items():
        assert np.allclose(v, z["g_" + k], rtol=0, atol=1e-11), k


# --------------------------------------------------------------------------- GPU

def _t(a, dtype=torch.float32):
    return torch.tensor(np.asarray(a), dtype=dtype, device="cuda")


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["sinkhorn_20.npz", "sinkhorn_7.npz"])
def test_hip_matches_golden_sinkhorn(name):
    import mhc

    z = load(name)
    M = _t(z["M"]).requires_grad_(True)
    P = mhc.sinkhorn_knopp(M, int(z["iters"]), float(z["eps"]))
    P.backward(_t(z["dP"]))
    assert rel_err(to_np(P), z["P"]) < FWD
    assert rel_err(to_np(M.grad), z["dM"]) < GRAD


@pytest.mark.gpu
def test_hip_matches_golden_dynamic_weights():
    import mhc

    z = load("dynamic_weights.npz")
    x, phi, bias = (_t(z[k]).requires_grad_(True) for k in ("x", "phi", "bias"))
    al = [_t([a]).requires_grad_(True) for a in z["alphas"]]
    out = mhc.fused_dynamic_weights(x, phi, bias, *al, 20, 1e-6)
    torch.autograd.backward(out, [_t(z["gH_pre"]), _t(z["gH_post"]), _t(z["gH_res"])])
    for o, k in zip(out, ("H_pre", "H_post", "H_res")):
        assert rel_err(to_np(o), z[k]) < FWD, k
    for t, k in ((x, "gx"), (phi, "gphi"), (bias, "gbias")):
        assert rel_err(to_np(t.grad), z[k]) < GRAD, k
    assert rel_err(np.array([to_np(a.grad)[0] for a in al]), z["galpha"]) < GRAD


@pytest.mark.gpu
def test_hip_matches_golden_stream_ops():
    import mhc

    z = load("stream_ops.npz")
    H, pre, res = (_t(z[k]).requires_grad_(True) for k in ("H", "H_pre", "H_res"))
    bi, hr = mhc.fused_stream_mix(H, pre, res)
    torch.autograd.backward([bi, hr], [_t(z["d_bi"]), _t(z["d_hr"])])
    assert rel_err(to_np(bi), z["bi"]) < FWD and rel_err(to_np(hr), z["hr"]) < FWD
    for t, k in ((H, "dH"), (pre, "dpre"), (res, "dres")):
        assert rel_err(to_np(t.grad), z[k]) < GRAD, k
    hr2, bo, post = (_t(z[k]).requires_grad_(True) for k in ("hr", "bo", "H_post"))
    H_new = mhc.fused_add_residual(hr2, bo, post)
    H_new.backward(_t(z["dHn"]))
    assert rel_err(to_np(H_new), z["H_new"]) < FWD
    assert rel_err(to_np(hr2.grad), z["dHn"]) < GRAD
    assert rel_err(to_np(bo.grad), z["d_bo"]) < GRAD and rel_err(to_np(post.grad), z["dpost"]) < GRAD


@pytest.mark.gpu
@pytest.mark.parametrize("name", LAYERS)
def test_hip_matches_golden_layer(name):
    import mhc

    z = load(name)
    dynamic, fused = layer_flags(name)
    D = z["H"].shape[-1]
    hc = mhc.HyperConnection(D, dynamic=dynamic, use_fused_weights=fused, layer_idx=1)
    with torch.no_grad():
        for n, prm in hc.named_parameters():
            prm.copy_(torch.tensor(z["p_" + n.replace(".weight", "")], dtype=torch.float32))
    hc = hc.cuda()
    H = _t(z["H"]).requires_grad_(True)
    bo = _t(z["bo"]).requires_grad_(True)
    bi, add = hc(H)
    H_new = add(bo)
    torch.autograd.backward([H_new, bi], [_t(z["dHn"]), _t(z["dbi"])])
    assert rel_err(to_np(bi), z["bi"]) < FWD and rel_err(to_np(H_new), z["H_new"]) < FWD
    assert rel_err(to_np(H.grad), z["g_H"]) < GRAD and rel_err(to_np(bo.grad), z["g_bo"]) < GRAD
    for n, prm in hc.named_parameters():
        ref = z["g_" + n]
        assert rel_err(to_np(prm.grad).reshape(ref.shape), ref) < GRAD, n
