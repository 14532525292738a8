"""Pins the CPU oracle (oracle/mhc_oracle.py) before anything is checked against it.

Each function is pinned by something other than its own formula:
closed forms and known answers, invariants the mathematics fixes,
an independent algorithm (Sinkhorn scaling vectors), central finite
differences in float64, and torch autograd of the independent torch
restatement in oracle/torch_path.py.  Each check is chosen so that a plausible
slip (eps in the wrong place, sum instead of mean in the RMS, swapped groups,
a missing x2, a transposed H_res, sgn(0) = +1) fails it.
"""

import numpy as np
import pytest
import torch

from helpers import rel_err
from oracle import mhc_oracle as O
from oracle import torch_path as TP

RNG = np.random.default_rng(1234)


def _fd(f, x, h=1e-6):
    """Central finite-difference gradient of scalar f at x (float64)."""
    g = np.zeros_like(x)
    it = np.nditer(x, flags=["multi_index"])
    for _ in it:
        i = it.multi_index
        old = x[i]
        x[i] = old + h
        fp = f(x)
        x[i] = old - h
        fm = f(x)
        x[i] = old
        g[i] = (fp - fm) / (2 * h)
    return g


# --------------------------------------------------------------------------- Sinkhorn forward

def test_sinkhorn_rank_one_gives_uniform():
    u = RNG.uniform(0.1, 3, size=(8, 4, 1))
    v = RNG.uniform(0.1, 3, size=(8, 1, 4))
    P = O.sinkhorn(u * v, iters=1, eps=0.0)
    assert np.abs(P - 0.25).max() < 1e-15
    P = O.sinkhorn(u * v, iters=1, eps=1e-8)
    assert np.abs(P - 0.25).max() < 1e-7


@pytest.mark.parametrize("eps", [1e-2, 1e-8])
def test_sinkhorn_all_equal_closed_form(eps):
    # M = c J: every entry follows a -> a/(4a + eps) twice per round, starting at |c| + eps.
    c = -1.7
    iters = 5
    a = abs(c) + eps
    for _ in range(iters):
        a = a / (4 * a + eps)
        a = a / (4 * a + eps)
    P = O.sinkhorn(np.full((1, 4, 4), c), iters, eps)
    assert np.abs(P - a).max() < 1e-15


def test_sinkhorn_doubly_stochastic_fixed_point():
    I = np.eye(4)
    perm = np.roll(I, 1, axis=1)
    A = 0.5 * I + 0.3 * perm + 0.2 * (perm @ perm)
    P = O.sinkhorn(A[None], iters=7, eps=0.0)
    assert np.abs(P[0] - A).max() < 1e-15


def test_sinkhorn_permutation_equivariance():
    M = RNG.standard_normal((16, 4, 4))
    p, q = RNG.permutation(4), RNG.permutation(4)
    P1 = O.sinkhorn(M[:, p][:, :, q], 20, 1e-3)
    P2 = O.sinkhorn(M, 20, 1e-3)[:, p][:, :, q]
    assert np.abs(P1 - P2).max() < 1e-13


def test_sinkhorn_matches_scaling_vector_algorithm():
    # Classic Sinkhorn on the scaling vectors: r = 1/(A c), c = 1/(A^T r);
    # after t rounds the normalised matrix is diag(r) A diag(c) (eps = 0).
    A = np.abs(RNG.standard_normal((32, 4, 4))) + 0.05
    iters = 9
    r = np.ones((32, 4))
    c = np.ones((32, 4))
    for _ in range(iters):
        r = 1.0 / np.einsum("bij,bj->bi", A, c)
        c = 1.0 / np.einsum("bij,bi->bj", A, r)
    ref = r[:, :, None] * A * c[:, None, :]
    assert rel_err(O.sinkhorn(A, iters, 0.0), ref) < 1e-12


def test_sinkhorn_columns_exact_rows_not_always_converged():
    M = np.exp(RNG.standard_normal((1 << 15, 4, 4)))
    P = O.sinkhorn(M, 20, 1e-8)
    # the last step normalises columns: column sums are (s / (s + eps)) ~ 1
    assert np.abs(P.sum(-2) - 1).max() < 1e-7
    # rows are not: a fraction of log-normal matrices is still off by > 1e-5
    frac = float((np.abs(P.sum(-1) - 1).max(-1) > 1e-5).mean())
    assert 0.0 < frac < 0.05


# --------------------------------------------------------------------------- Sinkhorn backward

def test_sinkhorn_backward_finite_differences():
    M = RNG.standard_normal((3, 4, 4))
    M += np.sign(M) * 0.05  # keep away from the |.| kink
    dP = RNG.standard_normal((3, 4, 4))
    g = O.sinkhorn_backward(M, dP, 6, 1e-3)
    fd = _fd(lambda m: float((O.sinkhorn(m, 6, 1e-3) * dP).sum()), M.copy())
    assert rel_err(g, fd) < 1e-7


def test_sinkhorn_backward_matches_torch_autograd_including_zeros():
    M = RNG.standard_normal((64, 4, 4))
    M[0, 1, 2] = 0.0
    M[5, 3, 3] = 0.0
    dP = RNG.standard_normal((64, 4, 4))
    Mt = torch.tensor(M, requires_grad=True)
    TP.sinkhorn(Mt, 20, 1e-8).backward(torch.tensor(dP))
    g = O.sinkhorn_backward(M, dP, 20, 1e-8)
    assert rel_err(g, Mt.grad.numpy()) < 1e-10
    # sgn(0) = 0, as torch's abs backward
    assert g[0, 1, 2] == 0.0 and g[5, 3, 3] == 0.0


# --------------------------------------------------------------------------- dynamic weights

def _sig(z):
    return 1.0 / (1.0 + np.exp(-z))


def test_dynamic_weights_phi_zero_known_answer():
    R, K = 3, 64
    x = RNG.standard_normal((R, K))
    bias = RNG.standard_normal(24)
    eps = 1e-6
    H_pre, H_post, H_res = O.dynamic_weights(x, np.zeros((K, 24)), bias, 0.3, 0.4, 0.5, 20, eps)
    sp = _sig(bias[0:4])
    assert np.abs(H_pre - sp / (sp.sum() + eps)).max() < 1e-15
    assert np.abs(H_post - 2 * _sig(bias[4:8])).max() < 1e-15
    assert np.abs(H_res - O.sinkhorn(bias[8:24].reshape(1, 4, 4), 20, eps)).max() < 1e-15


def test_dynamic_weights_constant_x_known_answer():
    # x = c * ones(K), phi[:, j] = (j + 1) / K  =>  raw_j = c (j + 1),
    # rms = sqrt(mean(x^2) + eps) = sqrt(c^2 + eps) (a mean, not a sum, over K).
    R, K, c, eps = 2, 32, 2.5, 1e-6
    x = np.full((R, K), c)
    phi = np.tile((np.arange(24) + 1.0) / K, (K, 1))
    bias = np.linspace(-1, 1, 24)
    alphas = (0.3, 0.7, 1.1)
    H_pre, H_post, H_res = O.dynamic_weights(x, phi, bias, *alphas, iters=3, eps=eps)
    inv = 1.0 / np.sqrt(c * c + eps)
    s = np.array([alphas[0 if j < 4 else (1 if j < 8 else 2)] * inv * c * (j + 1) + bias[j] for j in range(24)])
    sp = _sig(s[0:4])
    assert np.abs(H_pre[0] - sp / (sp.sum() + eps)).max() < 1e-14
    assert np.abs(H_post[1] - 2 * _sig(s[4:8])).max() < 1e-14
    assert np.abs(H_res[0] - O.sinkhorn(s[8:24].reshape(4, 4), 3, eps)).max() < 1e-14


def _dyn_inputs(R=3, K=16):
    x = RNG.standard_normal((R, K))
    phi = 0.3 * RNG.standard_normal((K, 24))
    bias = RNG.standard_normal(24)
    return x, phi, bias, (0.7, -0.4, 1.3)


def test_dynamic_weights_backward_finite_differences():
    x, phi, bias, al = _dyn_inputs()
    R = x.shape[0]
    gp, gq, gr = RNG.standard_normal((R, 4)), RNG.standard_normal((R, 4)), RNG.standard_normal((R, 4, 4))
    iters, eps = 5, 1e-3

    def loss(x_, phi_, bias_, a_):
        hp, hq, hr = O.dynamic_weights(x_, phi_, bias_, *a_, iters=iters, eps=eps)
        return float((hp * gp).sum() + (hq * gq).sum() + (hr * gr).sum())

    gx, gphi, gbias, ga = O.dynamic_weights_backward(x, phi, bias, *al, gp, gq, gr, iters, eps)
    assert rel_err(gx, _fd(lambda v: loss(v, phi, bias, al), x.copy())) < 1e-6
    assert rel_err(gphi, _fd(lambda v: loss(x, v, bias, al), phi.copy())) < 1e-6
    assert rel_err(gbias, _fd(lambda v: loss(x, phi, v, al), bias.copy())) < 1e-6
    ga_fd = _fd(lambda v: loss(x, phi, bias, tuple(v)), np.array(al, dtype=np.float64))
    assert rel_err(np.array(ga), ga_fd) < 1e-6


def test_dynamic_weights_backward_matches_torch_autograd():
    x, phi, bias, al = _dyn_inputs(R=5, K=40)
    R = x.shape[0]
    gp, gq, gr = RNG.standard_normal((R, 4)), RNG.standard_normal((R, 4)), RNG.standard_normal((R, 4, 4))
    t = [torch.tensor(v, requires_grad=True) for v in (x, phi, bias)]
    ta = [torch.tensor([a], dtype=torch.float64, requires_grad=True) for a in al]
    outs = TP.dynamic_weights(*t, *ta, iters=20, eps=1e-6)
    torch.autograd.backward(list(outs), [torch.tensor(gp), torch.tensor(gq), torch.tensor(gr)])
    gx, gphi, gbias, ga = O.dynamic_weights_backward(x, phi, bias, *al, gp, gq, gr, 20, 1e-6)
    assert rel_err(gx, t[0].grad.numpy()) < 1e-10
    assert rel_err(gphi, t[1].grad.numpy()) < 1e-10
    assert rel_err(gbias, t[2].grad.numpy()) < 1e-10
    assert rel_err(np.array(ga), np.array([a.grad.item() for a in ta])) < 1e-10


def test_dynamic_weights_backward_default_init_zeros():
    # phi = 0: raw = 0, so the alpha and x gradients vanish exactly.
    R, K = 4, 32
    x = RNG.standard_normal((R, K))
    bias = np.concatenate([[1, 0, 0, 0], np.ones(4), np.eye(4).reshape(16)])
    g = [RNG.standard_normal((R, 4)), RNG.standard_normal((R, 4)), RNG.standard_normal((R, 4, 4))]
    gx, gphi, gbias, ga = O.dynamic_weights_backward(x, np.zeros((K, 24)), bias, .1, .1, .1, *g, 20, 1e-6)
    assert np.all(gx == 0) and all(v == 0 for v in ga)
    assert np.abs(gphi).max() > 0


# --------------------------------------------------------------------------- stream mix / add residual

def _mix_inputs(B=2, S=5, D=6):
    H = RNG.standard_normal((B, S, 4, D))
    H_pre = RNG.uniform(0, 1, (B, 4))
    H_res = RNG.uniform(0, 1, (B, 4, 4))
    return H, H_pre, H_res


def test_stream_mix_identities():
    H, H_pre, H_res = _mix_inputs()
    B = H.shape[0]
    bi, hr = O.stream_mix(H, np.tile(np.eye(4)[2], (B, 1)), np.tile(np.eye(4), (B, 1, 1)))
    assert np.array_equal(bi, H[:, :, 2]) and np.array_equal(hr, H)
    perm = np.eye(4)[[3, 0, 2, 1]]  # row n selects stream perm_idx[n]
    _, hr = O.stream_mix(H, H_pre, np.tile(perm, (B, 1, 1)))
    assert np.array_equal(hr, H[:, :, [3, 0, 2, 1]])


def test_stream_mix_backward_adjoint():
    H, H_pre, H_res = _mix_inputs()
    d_bi = RNG.standard_normal(H.shape[:2] + H.shape[3:])
    d_hr = RNG.standard_normal(H.shape)
    dH, dpre, dres = O.stream_mix_backward(d_bi, d_hr, H, H_pre, H_res)
    # linear in H:  <d_bi, bi(X)> + <d_hr, hr(X)> = <dH, X>
    X = RNG.standard_normal(H.shape)
    bi, hr = O.stream_mix(X, H_pre, H_res)
    assert abs((d_bi * bi).sum() + (d_hr * hr).sum() - (dH * X).sum()) < 1e-10
    # linear in the weights
    dq, dr = RNG.standard_normal(H_pre.shape), RNG.standard_normal(H_res.shape)
    bi, hr = O.stream_mix(H, dq, dr)
    assert abs((d_bi * bi).sum() - (dpre * dq).sum()) < 1e-10
    assert abs((d_hr * hr).sum() - (dres * dr).sum()) < 1e-10


def test_add_residual_identity_and_backward_adjoint():
    H, _, _ = _mix_inputs()
    B, S, _, D = H.shape
    bo = RNG.standard_normal((B, S, D))
    H_post = RNG.uniform(0, 2, (B, 4))
    assert np.array_equal(O.add_residual(H, bo, np.zeros((B, 4))), H)
    out = O.add_residual(np.zeros_like(H), bo, np.ones((B, 4)))
    assert np.array_equal(out, np.repeat(bo[:, :, None, :], 4, axis=2))
    dHn = RNG.standard_normal(H.shape)
    dHr, dbo, dpost = O.add_residual_backward(dHn, bo, H_post)
    assert dHr is not None and np.array_equal(dHr, dHn)
    X = RNG.standard_normal(bo.shape)
    assert abs((dHn * O.add_residual(np.zeros_like(H), X, H_post)).sum() - (dbo * X).sum()) < 1e-10
    Y = RNG.standard_normal(H_post.shape)
    assert abs((dHn * O.add_residual(np.zeros_like(H), bo, Y)).sum() - (dpost * Y).sum()) < 1e-10


def test_stream_expand_collapse_closed_forms_adjoint_and_autograd():
    B, S, D = 2, 5, 7
    x = RNG.standard_normal((B, S, D))
    Y = RNG.standard_normal((B, S, 4, D))
    for scale in (1.0, 0.25, -1.5):
        H = O.stream_expand(x, scale)
        assert H.shape == (B, S, 4, D)
        for k in range(4):
            assert np.array_equal(H[:, :, k, :], scale * x)
        assert np.allclose(O.stream_collapse(H, scale), 4 * scale * scale * x, rtol=1e-14, atol=0)
        # adjoint pair: <expand(x), Y> = <x, collapse(Y)>
        assert abs((O.stream_expand(x, scale) * Y).sum() - (x * O.stream_collapse(Y, scale)).sum()) < 1e-10
        # torch autograd of independent torch expressions
        xt = torch.tensor(x, requires_grad=True)
        Ht = torch.tensor(Y, requires_grad=True)
        (xt.unsqueeze(2).expand(B, S, 4, D) * scale * torch.tensor(Y)).sum().backward()
        (torch.einsum("bsnd->bsd", Ht) * scale * torch.tensor(x)).sum().backward()
        assert np.allclose(O.stream_expand_backward(Y, scale), xt.grad.numpy(), rtol=1e-13, atol=1e-13)
        assert np.allclose(O.stream_collapse_backward(x, scale), Ht.grad.numpy(), rtol=1e-13, atol=1e-13)
    assert np.allclose(O.stream_collapse(Y, 0.25), Y.mean(axis=2), rtol=1e-13, atol=1e-15)


# --------------------------------------------------------------------------- mean-pool, static and unfused weights

def test_mean_pool_closed_form_and_layout():
    """H[b,s,n,d] = b + s + 10 n + 100 d: the mean over s is b + (S-1)/2 + 10 n + 100 d, at
    flat index n*D + d (stream-major), which pins mean (not sum) and the flatten order."""
    B, S, D = 2, 7, 3
    b, s, n, d = np.meshgrid(np.arange(B), np.arange(S), np.arange(4), np.arange(D), indexing="ij")
    H = (b + s + 10 * n + 100 * d).astype(np.float64)
    x = O.mean_pool(H)
    assert x.shape == (B, 4 * D)
    for bb in range(B):
        for nn_ in range(4):
            for dd in range(D):
                assert x[bb, nn_ * D + dd] == bb + (S - 1) / 2 + 10 * nn_ + 100 * dd


def _sig(z):
    return 1.0 / (1.0 + np.exp(-z))


@pytest.mark.parametrize("layer_idx", [0, 3])
def test_static_weights_default_init_known_answer(layer_idx):
    """Default parameters (H_post_base = 1, H_pre_base = onehot, H_res_base = I): H_post is
    sigmoid(1) = 0.7310585786300049 with no factor 2, H_pre puts sigmoid(1) / (sigmoid(1) + 1.5 +
    1e-8) on the layer's stream and 0.5 / (...) elsewhere, and H_res is the Sinkhorn of I + 1e-8,
    which is I to 1e-8."""
    pre = np.zeros(4)
    pre[layer_idx % 4] = 1.0
    H_post, H_pre, H_res = O.static_weights(pre, np.ones(4), np.eye(4), B=3)
    assert H_post.shape == (3, 4) and H_pre.shape == (3, 4) and H_res.shape == (3, 4, 4)
    assert np.all(H_post == _sig(1.0)) and abs(_sig(1.0) - 0.7310585786300049) < 1e-16
    den = _sig(1.0) + 1.5 + 1e-8
    want = np.full(4, 0.5 / den)
    want[layer_idx % 4] = _sig(1.0) / den
    assert np.allclose(H_pre, want, rtol=1e-15, atol=0)
    assert np.abs(H_res - np.eye(4)).max() < 5e-8


def test_unfused_weights_with_zero_linears_equal_static():
    """With W_pre = W_post = W_res = 0 the unfused path cannot see x, and must equal the
    static path on the same bases (sigmoid H_post without x2, 1e-8 in the H_pre normalisation
    and in the Sinkhorn); a nonzero W_res must then move H_res."""
    B, K = 3, 8
    x = RNG.standard_normal((B, K))
    bq, bp, br = RNG.standard_normal(4), RNG.standard_normal(4), RNG.standard_normal((4, 4))
    Wq, Wp, Wr = np.zeros((4, K)), np.zeros((4, K)), np.zeros((16, K))
    got = O.unfused_weights(x, Wq, Wp, Wr, 0.3, 0.2, 0.1, bq, bp, br)
    want = O.static_weights(bq, bp, br, B)
    for g_, w_ in zip(got, want):
        assert np.allclose(g_, w_, rtol=1e-13, atol=1e-15)
    moved = O.unfused_weights(x, Wq, Wp, RNG.standard_normal((16, K)), 0.3, 0.2, 0.1, bq, bp, br)
    assert np.abs(moved[2] - want[2]).max() > 1e-3


def test_static_weights_backward_finite_differences():
    bq, bp, br = RNG.standard_normal(4), RNG.standard_normal(4), RNG.standard_normal((4, 4))
    B = 2
    gp, gq, gr = RNG.standard_normal((B, 4)), RNG.standard_normal((B, 4)), RNG.standard_normal((B, 4, 4))

    def loss(q, p_, r):
        Hp, Hq, Hr = O.static_weights(q, p_, r, B, iters=5)
        return float((Hp * gp).sum() + (Hq * gq).sum() + (Hr * gr).sum())

    g_q, g_p, g_r = O.static_weights_backward(bq, bp, br, gp, gq, gr, iters=5)
    assert rel_err(g_q, _fd(lambda v: loss(v, bp, br), bq.copy())) < 1e-6
    assert rel_err(g_p, _fd(lambda v: loss(bq, v, br), bp.copy())) < 1e-6
    assert rel_err(g_r, _fd(lambda v: loss(bq, bp, v), br.copy())) < 1e-6


def test_unfused_weights_backward_finite_differences():
    B, K = 2, 6
    x = RNG.standard_normal((B, K))
    args = {
        "W_pre": 0.3 * RNG.standard_normal((4, K)), "W_post": 0.3 * RNG.standard_normal((4, K)),
        "W_res": 0.3 * RNG.standard_normal((16, K)), "scale_pre": 0.3, "scale_post": 0.2, "scale_res": 0.4,
        "H_pre_base": RNG.standard_normal(4), "H_post_base": RNG.standard_normal(4),
        "H_res_base": RNG.standard_normal((4, 4)),
    }
    gp, gq, gr = RNG.standard_normal((B, 4)), RNG.standard_normal((B, 4)), RNG.standard_normal((B, 4, 4))
    order = ["W_pre", "W_post", "W_res", "scale_pre", "scale_post", "scale_res", "H_pre_base", "H_post_base",
             "H_res_base"]

    def loss(xx, a):
        Hp, Hq, Hr = O.unfused_weights(xx, *[a[k] for k in order], iters=5, eps=1e-6)
        return float((Hp * gp).sum() + (Hq * gq).sum() + (Hr * gr).sum())

    g = O.unfused_weights_backward(x, *[args[k] for k in order], gp, gq, gr, iters=5, eps=1e-6)
    assert rel_err(g["x"], _fd(lambda v: loss(v, args), x.copy())) < 1e-6
    for k in order:
        def f(v, k=k):
            a = dict(args)
            a[k] = v if np.ndim(args[k]) else float(v)
            return loss(x, a)
        want = _fd(f, np.array(args[k], dtype=np.float64).copy())
        assert rel_err(np.asarray(g[k]).reshape(np.shape(want)), want) < 1e-6, k


# --------------------------------------------------------------------------- whole layer

def _layer_params(dynamic, fused, D, rng, zero_phi=False):
    p = {
        "H_pre_base": rng.standard_normal(4),
        "H_post_base": rng.standard_normal(4),
        "H_res_base": rng.standard_normal((4, 4)),
    }
    if dynamic and fused:
        p["phi"] = np.zeros((4 * D, 24)) if zero_phi else 0.2 * rng.standard_normal((4 * D, 24))
        for k in ("alpha_pre", "alpha_post", "alpha_res"):
            p[k] = np.array([rng.uniform(0.05, 0.5)])
    elif dynamic:
        for k in ("W_pre", "W_post", "W_res"):
            p[k] = 0.2 * rng.standard_normal(((16 if k == "W_res" else 4), 4 * D))
        for k in ("scale_pre", "scale_post", "scale_res"):
            p[k] = np.array([rng.uniform(0.05, 0.5)])
    return p


def _torch_params(p):
    out = {}
    for k, v in p.items():
        out[k + ".weight" if k.startswith("W_") else k] = torch.tensor(v)
    return out


@pytest.mark.parametrize("dynamic,fused", [(True, True), (True, False), (False, True)])
def test_layer_matches_torch_autograd(dynamic, fused):
    B, S, D = 2, 5, 6
    p = _layer_params(dynamic, fused, D, RNG)
    H = RNG.standard_normal((B, S, 4, D))
    bo = RNG.standard_normal((B, S, D))
    dHn = RNG.standard_normal((B, S, 4, D))
    dbi = RNG.standard_normal((B, S, D))
    bi, Hn, cache = O.layer_forward(p, H, bo, dynamic, fused, iters=20, eps=1e-6)
    g = O.layer_backward(p, cache, dHn, dbi)
    tbi, tHn, tg = TP.layer_grads(_torch_params(p), torch.tensor(H), torch.tensor(bo), torch.tensor(dHn),
                                  torch.tensor(dbi), dynamic, fused, 20, 1e-6, torch.float64)
    assert rel_err(bi, tbi.numpy()) < 1e-12
    assert rel_err(Hn, tHn.numpy()) < 1e-12
    for k, v in tg.items():
        key = k if k in g else k.replace(".weight", "")
        assert rel_err(np.asarray(g[key]).reshape(v.shape), v.numpy()) < 1e-9, k


def test_layer_backward_finite_differences_dynamic():
    B, S, D = 2, 3, 2
    p = _layer_params(True, True, D, RNG)
    H = RNG.standard_normal((B, S, 4, D))
    bo = RNG.standard_normal((B, S, D))
    dHn = RNG.standard_normal((B, S, 4, D))
    dbi = RNG.standard_normal((B, S, D))

    def loss(pp, HH):
        bi, Hn, _ = O.layer_forward(pp, HH, bo, True, True, iters=4, eps=1e-6)
        return float((bi * dbi).sum() + (Hn * dHn).sum())

    _, _, cache = O.layer_forward(p, H, bo, True, True, iters=4, eps=1e-6)
    g = O.layer_backward(p, cache, dHn, dbi)
    assert rel_err(g["H"], _fd(lambda v: loss(p, v), H.copy())) < 1e-6
    for k in ("phi", "H_pre_base", "H_post_base", "H_res_base", "alpha_pre", "alpha_post", "alpha_res"):
        def f(v, k=k):
            q = dict(p)
            q[k] = v
            return loss(q, H)
        assert rel_err(np.asarray(g[k]).reshape(p[k].shape), _fd(f, p[k].astype(np.float64).copy())) < 1e-6, k


# --------------------------------------------------------------------------- product torch baselines

def test_product_torch_baselines_match_oracle():
    import mhc

    B, S, D = 2, 4, 8
    for dynamic, fused in [(True, True), (True, False), (False, True)]:
        hc = mhc.HyperConnectionTorch(D, dynamic=dynamic, use_fused_weights=fused).double()
        p = _layer_params(dynamic, fused, D, RNG)
        with torch.no_grad():
            for name, prm in hc.named_parameters():
                prm.copy_(torch.tensor(p[name.replace(".weight", "")]).reshape(prm.shape))
        H = RNG.standard_normal((B, S, 4, D))
        bo = RNG.standard_normal((B, S, D))
        bi, add = hc(torch.tensor(H))
        Hn = add(torch.tensor(bo))
        obi, oHn, _ = O.layer_forward(p, H, bo, dynamic, fused)
        assert rel_err(bi.detach().numpy(), obi) < 1e-12
        assert rel_err(Hn.detach().numpy(), oHn) < 1e-12


# --------------------------------------------------------------------------- closed-form layer pins
#
# Structured inputs for which every weight has a closed form computed here from scalars, with no
# call into the oracle's own weight functions:
#
# * H[b, s, n, d] = c_b + delta_b * (-1)^s with S even, so the mean over the sequence is exactly c_b
#   and x = c_b * ones(4D);
# * every projection column (phi[:, j], or a Linear row) is v_j / (4D) * ones, so x . column = c_b v_j;
# * H_res logits of the form a * C + b * (J - C), where C is the cyclic shift C[n, (n+1) % 4] = 1
#   and J the all-ones matrix.  Every row and column of |a| C + |b| (J - C) + eps sums to the same r,
#   so each Sinkhorn normalisation only rescales the matrix: t -> t / (t r + eps).  C is not
#   symmetric, so a transposed H_res or a column-major flatten fails.
#
# RMS with the mean over K and eps inside the sqrt (module.py:145, _torch_baseline.py:78-80) is
# separated from a sum over K or eps outside the sqrt by c = 1e-3, where c^2 equals eps = 1e-6.

_C = np.roll(np.eye(4), 1, axis=1)
_J = np.ones((4, 4))


def _sk_closed(a, b, iters, eps):
    """Sinkhorn of a C + b (J - C), in closed form."""
    A, Bv = abs(a) + eps, abs(b) + eps
    r = A + 3 * Bv
    t = 1.0
    for _ in range(2 * iters):
        t = t / (t * r + eps)
    return t * (A * _C + Bv * (_J - _C))


def _sig1(z):
    return 1.0 / (1.0 + np.exp(-np.asarray(z, dtype=np.float64)))


def test_sinkhorn_cyclic_closed_form():
    """The helper itself against the oracle's Sinkhorn: a pin both ways, on a matrix whose
    answer is also known without iteration (a C + b (J - C) is doubly stochastic up to scale)."""
    a, b = 2.0, 0.5
    for iters, eps in [(1, 0.0), (20, 1e-8), (7, 1e-6)]:
        got = O.sinkhorn((a * _C + b * (_J - _C))[None], iters, eps)[0]
        assert np.abs(got - _sk_closed(a, b, iters, eps)).max() < 1e-15
    assert np.abs(_sk_closed(a, b, 20, 0.0) - (a * _C + b * (_J - _C)) / (a + 3 * b)).max() < 1e-15


def _structured_H(c, S, D, rng):
    B = len(c)
    sign = np.where(np.arange(S) % 2 == 0, 1.0, -1.0)[None, :, None, None]
    delta = rng.uniform(0.5, 2.0, size=(B, 1, 4, D))
    return np.asarray(c, dtype=np.float64)[:, None, None, None] + delta * sign


def _mix_and_add(H, bo, hpre, hpost, hres):
    """bi[b,s,d] = sum_n hpre[b,n] H[b,s,n,d];  H_new[b,s,n,d] = sum_m hres[b,n,m] H[b,s,m,d]
    + hpost[b,n] bo[b,s,d]  (_torch_baseline.py:136,141,164), written as explicit loops."""
    B, S, n, D = H.shape
    bi = np.zeros((B, S, D))
    Hn = np.zeros_like(H)
    for b in range(B):
        for i in range(4):
            bi[b] += hpre[b][i] * H[b, :, i]
            Hn[b, :, i] = hpost[b][i] * bo[b]
            for m in range(4):
                Hn[b, :, i] += hres[b][i][m] * H[b, :, m]
    return bi, Hn


@pytest.mark.parametrize("layer_idx", [0, 2])
def test_layer_static_known_answer(layer_idx):
    """Static layer (module.py:108-117, 170-180): H_post = sigmoid(b_post) with no x2, H_pre =
    sigmoid(b_pre) / (sum + 1e-8), H_res = Sinkhorn(b_res, eps 1e-8); bi uses H_pre, the closure
    uses H_res on H and H_post on branch_output."""
    rng = np.random.default_rng(7 + layer_idx)
    B, S, D = 2, 4, 3
    bq = np.array([0.3, -0.7, 1.2, 0.1])
    bq[layer_idx] += 1.0
    bp = np.array([-0.4, 0.9, 0.2, 1.5])
    a, b = 2.0, -0.5
    p = {"H_pre_base": bq, "H_post_base": bp, "H_res_base": a * _C + b * (_J - _C)}
    H = rng.standard_normal((B, S, 4, D))
    bo = rng.standard_normal((B, S, D))
    bi, Hn, _ = O.layer_forward(p, H, bo, dynamic=False, iters=20)
    sq = _sig1(bq)
    hpre = np.tile(sq / (sq.sum() + 1e-8), (B, 1))
    hpost = np.tile(_sig1(bp), (B, 1))
    hres = np.tile(_sk_closed(a, b, 20, 1e-8), (B, 1, 1))
    want_bi, want_Hn = _mix_and_add(H, bo, hpre, hpost, hres)
    assert np.abs(bi - want_bi).max() < 1e-13
    assert np.abs(Hn - want_Hn).max() < 1e-13


def test_layer_dynamic_default_init_known_answer():
    """Fused dynamic layer at phi = 0 (the default init): s = bias = [b_pre, b_post, b_res]
    (module.py:127-131), H_pre = sigmoid(b_pre) / (sum + 1e-6), H_post = 2 sigmoid(b_post),
    H_res = Sinkhorn(|b_res| + 1e-6, eps 1e-6).  A pre/post bias swap, a missing x2, the weights
    returned as (H_pre, H_post) instead of (H_post, H_pre), or a transposed H_res fail."""
    rng = np.random.default_rng(11)
    B, S, D = 2, 4, 3
    bq, bp = np.array([1.0, 0.0, -0.3, 0.6]), np.array([1.0, -1.2, 0.4, 0.8])
    a, b = 1.5, 0.25
    p = {"H_pre_base": bq, "H_post_base": bp, "H_res_base": a * _C + b * (_J - _C),
         "phi": np.zeros((4 * D, 24)), "alpha_pre": np.array([0.3]), "alpha_post": np.array([0.2]),
         "alpha_res": np.array([0.1])}
    H = rng.standard_normal((B, S, 4, D))
    bo = rng.standard_normal((B, S, D))
    bi, Hn, _ = O.layer_forward(p, H, bo, dynamic=True, fused=True, iters=20, eps=1e-6)
    sq = _sig1(bq)
    hpre = np.tile(sq / (sq.sum() + 1e-6), (B, 1))
    hpost = np.tile(2.0 * _sig1(bp), (B, 1))
    hres = np.tile(_sk_closed(a, b, 20, 1e-6), (B, 1, 1))
    want_bi, want_Hn = _mix_and_add(H, bo, hpre, hpost, hres)
    assert np.abs(bi - want_bi).max() < 1e-13
    assert np.abs(Hn - want_Hn).max() < 1e-13


def _group_cols(v_pre, v_post, res_ab, K):
    """phi [K, 24] whose column j is v_j / K * ones; the H_res group is a C + b (J - C), row-major."""
    v = np.concatenate([v_pre, v_post, (res_ab[0] * _C + res_ab[1] * (_J - _C)).reshape(16)])
    return np.tile(v / K, (K, 1))


def test_layer_dynamic_structured_phi_known_answer():
    """Fused dynamic layer with phi != 0 on the structured inputs.  x = c_b ones (the sequence
    mean), raw_j = c_b v_j, inv_rms = 1 / sqrt(c_b^2 + eps), s_j = alpha_g inv_rms raw_j + bias_j with
    alpha_pre on columns 0:4, alpha_post on 4:8 and alpha_res on 8:24 (_torch_baseline.py:73-111).
    c = 1e-3 sits where eps inside / outside the sqrt differ; c = 0.5 where mean / sum over K and
    over S differ."""
    rng = np.random.default_rng(5)
    S, D = 6, 2
    K = 4 * D
    c = np.array([1e-3, 0.5])
    B = len(c)
    eps, iters = 1e-6, 20
    vq, vp = np.array([0.5, -1.0, 2.0, 0.3]), np.array([-0.6, 1.1, 0.0, 0.9])
    res_ab = (3.0, -1.0)
    bq, bp = np.array([0.2, -0.1, 0.4, 0.0]), np.array([0.7, -0.3, 0.1, 0.5])
    base_ab = (1.0, 0.2)
    ap, aq, ar = 0.7, 0.4, 0.25
    p = {"H_pre_base": bq, "H_post_base": bp, "H_res_base": base_ab[0] * _C + base_ab[1] * (_J - _C),
         "phi": _group_cols(vq, vp, res_ab, K), "alpha_pre": np.array([ap]), "alpha_post": np.array([aq]),
         "alpha_res": np.array([ar])}
    H = _structured_H(c, S, D, rng)
    bo = rng.standard_normal((B, S, D))
    bi, Hn, cache = O.layer_forward(p, H, bo, dynamic=True, fused=True, iters=iters, eps=eps)
    assert np.abs(cache["x"] - c[:, None]).max() < 1e-15
    hpre, hpost, hres = [], [], []
    for cb in c:
        k = cb / np.sqrt(cb * cb + eps)
        sq = _sig1(ap * k * vq + bq)
        hpre.append(sq / (sq.sum() + eps))
        hpost.append(2.0 * _sig1(aq * k * vp + bp))
        hres.append(_sk_closed(base_ab[0] + ar * k * res_ab[0], base_ab[1] + ar * k * res_ab[1], iters, eps))
    want_bi, want_Hn = _mix_and_add(H, bo, hpre, hpost, hres)
    assert rel_err(bi, want_bi) < 1e-13
    assert rel_err(Hn, want_Hn) < 1e-13
    # the chosen inputs do separate the slips named above
    k_sum = c[0] / np.sqrt(K * c[0] ** 2 + eps)
    k_out = c[0] / (abs(c[0]) + eps)
    k_in = c[0] / np.sqrt(c[0] ** 2 + eps)
    assert abs(k_sum - k_in) > 0.1 and abs(k_out - k_in) > 0.2


def test_unfused_weights_structured_known_answer():
    """Unfused path (module.py:143-163): rms = sqrt(mean(x^2) + eps), x_n = x / rms, each logit is
    base + scale * (W x_n), H_post = sigmoid (no x2), 1e-8 in the H_pre normalisation and in the
    Sinkhorn.  Linears whose rows are w_i / K * ones give W x_n = w_i c / sqrt(c^2 + eps) for
    x = c ones.  A sum-RMS, eps outside the sqrt, or the scale applied before the normalisation
    (where the RMS would cancel it) fail at c = 1e-3 or c = 0.5."""
    K, eps, iters = 8, 1e-6, 20
    wq, wp = np.array([0.5, -1.0, 2.0, 0.3]), np.array([-0.6, 1.1, 0.0, 0.9])
    res_ab = (3.0, -1.0)
    Wq, Wp = np.tile(wq[:, None] / K, (1, K)), np.tile(wp[:, None] / K, (1, K))
    Wr = np.tile((res_ab[0] * _C + res_ab[1] * (_J - _C)).reshape(16, 1) / K, (1, K))
    sq_, sp_, sr_ = 0.4, 0.7, 0.25
    bq, bp = np.array([0.2, -0.1, 0.4, 0.0]), np.array([0.7, -0.3, 0.1, 0.5])
    base_ab = (1.0, 0.2)
    br = base_ab[0] * _C + base_ab[1] * (_J - _C)
    c = np.array([1e-3, 0.5])
    x = np.tile(c[:, None], (1, K))
    H_post, H_pre, H_res = O.unfused_weights(x, Wq, Wp, Wr, sq_, sp_, sr_, bq, bp, br, iters, eps)
    for i, cb in enumerate(c):
        k = cb / np.sqrt(cb * cb + eps)
        assert np.abs(H_post[i] - _sig1(bp + sp_ * k * wp)).max() < 1e-15
        sq = _sig1(bq + sq_ * k * wq)
        assert np.abs(H_pre[i] - sq / (sq.sum() + 1e-8)).max() < 1e-15
        want = _sk_closed(base_ab[0] + sr_ * k * res_ab[0], base_ab[1] + sr_ * k * res_ab[1], iters, 1e-8)
        assert np.abs(H_res[i] - want).max() < 1e-14


def test_layer_unfused_structured_known_answer():
    """The unfused layer end to end on the structured H: the sequence mean feeds the RMS, bi uses
    H_pre and the closure H_res and H_post (module.py:165-180)."""
    rng = np.random.default_rng(9)
    S, D = 4, 2
    K = 4 * D
    c = np.array([1e-3, 0.5])
    B = len(c)
    eps, iters = 1e-6, 20
    wq, wp = np.array([0.5, -1.0, 2.0, 0.3]), np.array([-0.6, 1.1, 0.0, 0.9])
    res_ab, base_ab = (3.0, -1.0), (1.0, 0.2)
    p = {"H_pre_base": np.array([0.2, -0.1, 0.4, 0.0]), "H_post_base": np.array([0.7, -0.3, 0.1, 0.5]),
         "H_res_base": base_ab[0] * _C + base_ab[1] * (_J - _C),
         "W_pre": np.tile(wq[:, None] / K, (1, K)), "W_post": np.tile(wp[:, None] / K, (1, K)),
         "W_res": np.tile((res_ab[0] * _C + res_ab[1] * (_J - _C)).reshape(16, 1) / K, (1, K)),
         "scale_pre": np.array([0.4]), "scale_post": np.array([0.7]), "scale_res": np.array([0.25])}
    H = _structured_H(c, S, D, rng)
    bo = rng.standard_normal((B, S, D))
    bi, Hn, _ = O.layer_forward(p, H, bo, dynamic=True, fused=False, iters=iters, eps=eps)
    hpre, hpost, hres = [], [], []
    for cb in c:
        k = cb / np.sqrt(cb * cb + eps)
        sq = _sig1(p["H_pre_base"] + 0.4 * k * wq)
        hpre.append(sq / (sq.sum() + 1e-8))
        hpost.append(_sig1(p["H_post_base"] + 0.7 * k * wp))
        hres.append(_sk_closed(base_ab[0] + 0.25 * k * res_ab[0], base_ab[1] + 0.25 * k * res_ab[1], iters, 1e-8))
    want_bi, want_Hn = _mix_and_add(H, bo, hpre, hpost, hres)
    assert rel_err(bi, want_bi) < 1e-13
    assert rel_err(Hn, want_Hn) < 1e-13


@pytest.mark.parametrize("dynamic,fused", [(True, False), (False, True)])
def test_layer_backward_finite_differences_static_and_unfused(dynamic, fused):
    """The whole layer's gradients against central differences of its forward, for the paths
    the dynamic-fused FD test does not cover."""
    rng = np.random.default_rng(21)
    B, S, D = 2, 3, 2
    p = _layer_params(dynamic, fused, D, rng)
    H = rng.standard_normal((B, S, 4, D))
    bo = rng.standard_normal((B, S, D))
    dHn = rng.standard_normal((B, S, 4, D))
    dbi = rng.standard_normal((B, S, D))

    def loss(pp, HH, bb):
        bi, Hn, _ = O.layer_forward(pp, HH, bb, dynamic, fused, iters=4, eps=1e-6)
        return float((bi * dbi).sum() + (Hn * dHn).sum())

    _, _, cache = O.layer_forward(p, H, bo, dynamic, fused, iters=4, eps=1e-6)
    g = O.layer_backward(p, cache, dHn, dbi)
    assert rel_err(g["H"], _fd(lambda v: loss(p, v, bo), H.copy())) < 1e-6
    assert rel_err(g["bo"], _fd(lambda v: loss(p, H, v), bo.copy())) < 1e-6
    for k in p:
        def f(v, k=k):
            q = dict(p)
            q[k] = v
            return loss(q, H, bo)
        key = k + ".weight" if k.startswith("W_") else k
        assert rel_err(np.asarray(g[key]).reshape(p[k].shape), _fd(f, p[k].astype(np.float64).copy())) < 1e-6, k
