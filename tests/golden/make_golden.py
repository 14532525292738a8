"""Writes the golden fixtures in this directory from the float64 CPU oracle.

    python tests/golden/make_golden.py

Each fixture is a small .npz (numpy, no pickles) of seeded inputs and the
oracle's outputs and gradients, in float64.  The reference ships no golden
vectors (its tests compute references on the fly), so these freeze the oracle
(oracle/mhc_oracle.py), which tests/test_oracle.py pins independently.
tests/test_golden.py checks that the oracle still reproduces them (CPU) and
that the HIP path matches them (GPU).
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import mhc_oracle as O  # noqa: E402


def sinkhorn_case(rng, iters, eps):
    M = rng.standard_normal((16, 4, 4))
    M[0, 1, 2] = 0.0          # exact zero: sgn(0) = 0 in the backward
    M[3] = np.exp(rng.standard_normal((4, 4)))
    dP = rng.standard_normal((16, 4, 4))
    return dict(M=M, dP=dP, iters=np.int64(iters), eps=np.float64(eps),
                P=O.sinkhorn(M, iters, eps), dM=O.sinkhorn_backward(M, dP, iters, eps))


def dynw_case(rng):
    R, K = 3, 64
    x = rng.standard_normal((R, K))
    phi = rng.standard_normal((K, 24)) * 0.3
    bias = rng.standard_normal(24)
    alphas = np.array([0.7, -0.4, 1.3])
    gp, gq, gr = rng.standard_normal((R, 4)), rng.standard_normal((R, 4)), rng.standard_normal((R, 4, 4))
    H_pre, H_post, H_res = O.dynamic_weights(x, phi, bias, *alphas, 20, 1e-6)
    gx, gphi, gbias, ga = O.dynamic_weights_backward(x, phi, bias, *alphas, gp, gq, gr, 20, 1e-6)
    return dict(x=x, phi=phi, bias=bias, alphas=alphas, gH_pre=gp, gH_post=gq, gH_res=gr,
                H_pre=H_pre, H_post=H_post, H_res=H_res, gx=gx, gphi=gphi, gbias=gbias, galpha=np.array(ga))


def mix_case(rng):
    B, S, D = 2, 5, 8
    H = rng.standard_normal((B, S, 4, D))
    z = rng.standard_normal((B, 4))
    H_pre = np.exp(z) / np.exp(z).sum(-1, keepdims=True)
    H_res = O.sinkhorn(rng.standard_normal((B, 4, 4)), 20, 1e-8)
    H_post = rng.uniform(0, 2, (B, 4))
    bo = rng.standard_normal((B, S, D))
    d_bi = rng.standard_normal((B, S, D))
    d_hr = rng.standard_normal((B, S, 4, D))
    dHn = rng.standard_normal((B, S, 4, D))
    bi, hr = O.stream_mix(H, H_pre, H_res)
    dH, dpre, dres = O.stream_mix_backward(d_bi, d_hr, H, H_pre, H_res)
    H_new = O.add_residual(hr, bo, H_post)
    _, d_bo, dpost = O.add_residual_backward(dHn, bo, H_post)
    return dict(H=H, H_pre=H_pre, H_res=H_res, H_post=H_post, bo=bo, d_bi=d_bi, d_hr=d_hr, dHn=dHn,
                bi=bi, hr=hr, dH=dH, dpre=dpre, dres=dres, H_new=H_new, d_bo=d_bo, dpost=dpost)


def layer_case(rng, dynamic, fused, phi_std):
    B, S, D = 2, 6, 8
    p = {"H_post_base": np.ones(4), "H_pre_base": np.eye(4)[1], "H_res_base": np.eye(4)}
    if not dynamic:
        p["H_res_base"] = rng.standard_normal((4, 4))
    elif fused:
        p["phi"] = rng.standard_normal((4 * D, 24)) * phi_std
        for k in ("alpha_pre", "alpha_post", "alpha_res"):
            p[k] = np.array([0.1])
    else:
        p["W_post"] = rng.standard_normal((4, 4 * D)) * phi_std
        p["W_pre"] = rng.standard_normal((4, 4 * D)) * phi_std
        p["W_res"] = rng.standard_normal((16, 4 * D)) * phi_std
        for k in ("scale_pre", "scale_post", "scale_res"):
            p[k] = np.array([0.1])
    H = rng.standard_normal((B, S, 4, D))
    bo = rng.standard_normal((B, S, D))
    dHn = rng.standard_normal((B, S, 4, D))
    dbi = rng.standard_normal((B, S, D))
    bi, H_new, cache = O.layer_forward(p, H, bo, dynamic, fused, 20, 1e-6)
    g = O.layer_backward(p, cache, dHn, dbi)
    out = {"H": H, "bo": bo, "dHn": dHn, "dbi": dbi, "bi": bi, "H_new": H_new}
    out.update({"p_" + k: v for k, v in p.items()})
    out.update({"g_" + k: v for k, v in g.items()})
    return out


def main():
    rng = np.random.default_rng(20261201)
    cases = {
        "sinkhorn_20.npz": sinkhorn_case(rng, 20, 1e-8),
        "sinkhorn_7.npz": sinkhorn_case(rng, 7, 1e-3),
        "dynamic_weights.npz": dynw_case(rng),
        "stream_ops.npz": mix_case(rng),
        "layer_dynamic_init.npz": layer_case(rng, True, True, 0.0),
        "layer_dynamic.npz": layer_case(rng, True, True, 0.3),
        "layer_static.npz": layer_case(rng, False, True, 0.0),
        "layer_unfused.npz": layer_case(rng, True, False, 0.3),
    }
    for name, arrays in cases.items():
        np.savez(os.path.join(HERE, name), **arrays)
        print(name, sum(np.asarray(v).nbytes for v in arrays.values()), "bytes")


if __name__ == "__main__":
    main()
