"""The Sinkhorn backward's scaled-coordinate form, restated in float64 numpy
and held to the oracle's explicit backward (no GPU).

The HIP backward (sk_backward_scaled / sk_backward_segmented in
mhc-triton_amd/csrc/sinkhorn.hpp) runs the forward as P_t = P0 * u_t v_t^T and
carries the adjoint as g = dP * u v^T.  Column normalisation of round t then
reads g -= u_{t+1,i} v_{t+1,j} sum_k g_kj P0_kj and row normalisation
g -= v_{t,j} u_{t+1,i} sum_l g_il P0_il, which rests on c_j v_{t,j} = v_{t+1,j}
and r_i u_{t,i} = u_{t+1,i}.  In exact arithmetic this is the explicit
backward of the reference's loop (src/mhc/_backward.py:30-262 as restated in
oracle.sinkhorn_backward); in float64 the two agree to rounding, so a dropped
scale, a swapped u / v index or a round off by one fails here."""

import numpy as np
import pytest

from oracle import mhc_oracle as O


def scaled_backward(M, dP, iters, eps):
    """One matrix set [N, 4, 4]: the kernel's algorithm in float64."""
    p0 = np.abs(M) + eps
    n = M.shape[0]
    U = [np.ones((n, 4))]
    V = [np.ones((n, 4))]
    w = np.ones((n, 4))
    z = np.ones((n, 4))
    for _ in range(iters):
        w = eps * w + np.einsum("nij,nj->ni", p0, V[-1])
        U.append(1.0 / w)
        z = eps * z + np.einsum("ni,nij->nj", U[-1], p0)
        V.append(1.0 / z)
    g = dP * U[iters][:, :, None] * V[iters][:, None, :]
    for t in range(iters - 1, -1, -1):
        e = np.einsum("nij,nij->nj", g, p0) * V[t + 1]
        g = g - U[t + 1][:, :, None] * e[:, None, :]
        f = np.einsum("nij,nij->ni", g, p0) * U[t + 1]
        g = g - V[t][:, None, :] * f[:, :, None]
    return g * np.sign(M)


@pytest.mark.parametrize("iters", [0, 1, 2, 7, 20, 33])
def test_scaled_adjoint_equals_explicit_backward(iters):
    rng = np.random.default_rng(iters)
    M = np.exp(rng.standard_normal((64, 4, 4))) * rng.choice([-1.0, 1.0], (64, 4, 4))
    M[0, 0, 0] = 0.0
    M[3] = rng.standard_normal((4, 4)) * 1e-3  # entries near eps's scale
    dP = rng.standard_normal((64, 4, 4))
    for eps in (1e-8, 1e-6, 1e-2):
        ref = O.sinkhorn_backward(M, dP, iters, eps)
        got = scaled_backward(M, dP, iters, eps)
        assert np.max(np.abs(got - ref)) <= 1e-10 * max(np.max(np.abs(ref)), 1e-300)
        assert got[0, 0, 0] == 0.0


def test_scaled_forward_vectors_reproduce_the_explicit_state():
    """P0 * u_t v_t^T after t rounds is the oracle's state after t rounds."""
    rng = np.random.default_rng(5)
    M = np.exp(rng.standard_normal((16, 4, 4)))
    eps = 1e-6
    p0 = np.abs(M) + eps
    u = np.ones((16, 4))
    v = np.ones((16, 4))
    w = np.ones((16, 4))
    z = np.ones((16, 4))
    for t in range(1, 9):
        w = eps * w + np.einsum("nij,nj->ni", p0, v)
        u = 1.0 / w
        z = eps * z + np.einsum("ni,nij->nj", u, p0)
        v = 1.0 / z
        P = p0 * u[:, :, None] * v[:, None, :]
        np.testing.assert_allclose(P, O.sinkhorn(M, t, eps), rtol=1e-12, atol=0)
