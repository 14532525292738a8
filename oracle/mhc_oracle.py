"""CPU oracle for the mHC hot path.  TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg import this module, and only as the checker: the product (``mhc`` on the
HIP library) never calls it.

A numpy restatement of the reference's pure-PyTorch path, computed in float64
by default (``dt=np.float32`` mimics an fp32 torch run), with explicit
reverse-mode gradients for every function.  Mixed dtypes follow one policy:
inputs are upcast to ``dt`` (the reference's own torch path raises on a bf16 H
with fp32 weights, ``_torch_baseline.py:136,141`` einsum dtype mismatch, so the
parity target for bf16/fp16 inputs is the fp32/fp64 math on the same values).

Reference citations are paths under src/mhc/ of WithNucleusAI/mHC-triton.
How each function is pinned (closed forms, invariants, finite differences,
torch autograd of an independent torch restatement) is in tests/test_oracle.py.
"""

from __future__ import annotations

import numpy as np

F64 = np.float64


def _a(x, dt):
    return np.asarray(x, dtype=dt)


def _s(x, dt):
    """A scalar parameter (a Python number or a one-element array) as dt."""
    return dt(np.asarray(x).reshape(-1)[0])


def sigmoid(z):
    return 1.0 / (1.0 + np.exp(-z))


# ---------------------------------------------------------------------------
# Sinkhorn-Knopp  (_torch_baseline.py:12-35; backward _backward.py:29-262)
# ---------------------------------------------------------------------------

def sinkhorn(M, iters=20, eps=1e-8, dt=F64):
    """P = |M| + eps, then `iters` rounds of P /= (rowsum + eps); P /= (colsum + eps)."""
    P = np.abs(_a(M, dt)) + dt(eps)
    for _ in range(iters):
        P = P / (P.sum(axis=-1, keepdims=True) + dt(eps))
        P = P / (P.sum(axis=-2, keepdims=True) + dt(eps))
    return P


def sinkhorn_backward(M, dP, iters=20, eps=1e-8, dt=F64):
    """dM for the cotangent dP.  Each normalisation y = x / (sum(x) + eps) has
    the vector-Jacobian product dx = (dy - <dy, y>) / (sum(x) + eps); the |M|
    step contributes sgn(M) with sgn(0) = 0 (torch autograd semantics; the
    reference Triton kernel uses +1 at 0, _backward.py:106-121)."""
    M = _a(M, dt)
    P = np.abs(M) + dt(eps)
    states = []
    for _ in range(iters):
        states.append(P)
        P = P / (P.sum(axis=-1, keepdims=True) + dt(eps))
        P = P / (P.sum(axis=-2, keepdims=True) + dt(eps))
    d = _a(dP, dt)
    for P0 in reversed(states):
        r = P0.sum(axis=-1, keepdims=True) + dt(eps)
        Pr = P0 / r
        c = Pr.sum(axis=-2, keepdims=True) + dt(eps)
        Pc = Pr / c
        d = (d - (d * Pc).sum(axis=-2, keepdims=True)) / c
        d = (d - (d * Pr).sum(axis=-1, keepdims=True)) / r
    return d * np.sign(M)


# ---------------------------------------------------------------------------
# Dynamic weights, Eq. 14-19  (_torch_baseline.py:38-111; backward ops.py:110-228)
# ---------------------------------------------------------------------------

GROUPS = (slice(0, 4), slice(4, 8), slice(8, 24))


def dynamic_weights(x, phi, bias, a_pre, a_post, a_res, iters=20, eps=1e-6, dt=F64):
    """Returns (H_pre [R,4], H_post [R,4], H_res [R,4,4])."""
    x, phi, bias = _a(x, dt), _a(phi, dt), _a(bias, dt)
    R, K = x.shape
    raw = x @ phi
    inv_rms = 1.0 / np.sqrt((x * x).sum(axis=-1, keepdims=True) / K + dt(eps))
    s = np.empty_like(raw)
    for g, a in zip(GROUPS, (a_pre, a_post, a_res)):
        s[:, g] = inv_rms * dt(a) * raw[:, g] + bias[g]
    sg = sigmoid(s[:, 0:4])
    H_pre = sg / (sg.sum(axis=-1, keepdims=True) + dt(eps))
    H_post = 2.0 * sigmoid(s[:, 4:8])
    H_res = sinkhorn(s[:, 8:24].reshape(R, 4, 4), iters, eps, dt)
    return H_pre, H_post, H_res


def dynamic_weights_backward(x, phi, bias, a_pre, a_post, a_res, gH_pre, gH_post, gH_res,
                             iters=20, eps=1e-6, dt=F64):
    """Gradients (gx, gphi, gbias[24], [g_a_pre, g_a_post, g_a_res]) for the
    cotangents of (H_pre, H_post, H_res); None cotangents count as zero."""
    x, phi, bias = _a(x, dt), _a(phi, dt), _a(bias, dt)
    R, K = x.shape
    alphas = [dt(a) for a in (a_pre, a_post, a_res)]
    raw = x @ phi
    rms = np.sqrt((x * x).sum(axis=-1, keepdims=True) / K + dt(eps))
    inv_rms = 1.0 / rms
    s = np.empty_like(raw)
    for g, a in zip(GROUPS, alphas):
        s[:, g] = inv_rms * a * raw[:, g] + bias[g]
    gH_pre = np.zeros((R, 4), dt) if gH_pre is None else _a(gH_pre, dt)
    gH_post = np.zeros((R, 4), dt) if gH_post is None else _a(gH_post, dt)
    gH_res = np.zeros((R, 4, 4), dt) if gH_res is None else _a(gH_res, dt).reshape(R, 4, 4)
    gs = np.empty_like(s)
    # H_res = Sinkhorn(s_res)
    gs[:, 8:24] = sinkhorn_backward(s[:, 8:24].reshape(R, 4, 4), gH_res, iters, eps, dt).reshape(R, 16)
    # H_post = 2 sigmoid(s_post)
    sq = sigmoid(s[:, 4:8])
    gs[:, 4:8] = gH_post * 2.0 * sq * (1.0 - sq)
    # H_pre = sigmoid(s_pre) / (sum + eps)
    sp = sigmoid(s[:, 0:4])
    den = sp.sum(axis=-1, keepdims=True) + dt(eps)
    H_pre = sp / den
    gsig = (gH_pre - (gH_pre * H_pre).sum(axis=-1, keepdims=True)) / den
    gs[:, 0:4] = gsig * sp * (1.0 - sp)
    # s = inv_rms * alpha * raw + bias
    graw = np.empty_like(raw)
    galpha = []
    g_inv = np.zeros((R, 1), dt)
    for g, a in zip(GROUPS, alphas):
        graw[:, g] = gs[:, g] * inv_rms * a
        galpha.append((gs[:, g] * inv_rms * raw[:, g]).sum())
        g_inv += (gs[:, g] * a * raw[:, g]).sum(axis=-1, keepdims=True)
    gbias = gs.sum(axis=0)
    # inv_rms = 1/rms, rms = sqrt(sum x^2 / K + eps)
    g_rms = g_inv * (-inv_rms * inv_rms)
    gx = graw @ phi.T + g_rms * x / (K * rms)
    gphi = x.T @ graw
    return gx, gphi, gbias, galpha


# ---------------------------------------------------------------------------
# Stream mix, Eq. 10-11  (_torch_baseline.py:114-143; backward _backward.py:358-496)
# ---------------------------------------------------------------------------

def stream_mix(H, H_pre, H_res, dt=F64):
    """branch_input [B,S,D] and H_residual [B,S,4,D]."""
    H, H_pre, H_res = _a(H, dt), _a(H_pre, dt), _a(H_res, dt)
    bi = np.einsum("bn,bsnd->bsd", H_pre, H)
    hr = np.einsum("bnm,bsmd->bsnd", H_res, H)
    return bi, hr


def stream_mix_backward(d_bi, d_hr, H, H_pre, H_res, dt=F64):
    """(dH, dH_pre, dH_res)."""
    d_bi, d_hr, H = _a(d_bi, dt), _a(d_hr, dt), _a(H, dt)
    H_pre, H_res = _a(H_pre, dt), _a(H_res, dt)
    dH = np.einsum("bm,bsd->bsmd", H_pre, d_bi) + np.einsum("bnm,bsnd->bsmd", H_res, d_hr)
    dH_pre = np.einsum("bsd,bsnd->bn", d_bi, H)
    dH_res = np.einsum("bsnd,bsmd->bnm", d_hr, H)
    return dH, dH_pre, dH_res


# ---------------------------------------------------------------------------
# Add residual, Eq. 12  (_torch_baseline.py:146-166; backward _backward.py:269-351)
# ---------------------------------------------------------------------------

def add_residual(H_residual, bo, H_post, dt=F64):
    H_residual, bo, H_post = _a(H_residual, dt), _a(bo, dt), _a(H_post, dt)
    return H_residual + H_post[:, None, :, None] * bo[:, :, None, :]


def add_residual_backward(dH_new, bo, H_post, dt=F64):
    """(dH_residual, d_bo, dH_post)."""
    dH_new, bo, H_post = _a(dH_new, dt), _a(bo, dt), _a(H_post, dt)
    d_bo = np.einsum("bn,bsnd->bsd", H_post, dH_new)
    dH_post = np.einsum("bsnd,bsd->bn", dH_new, bo)
    return dH_new, d_bo, dH_post


# ---------------------------------------------------------------------------
# Stream expand / collapse at the ends of a stack.  No reference function: the
# reference takes the (batch, seq, 4, dim) hyper-hidden state as given
# (README.md:38-39).  The two are adjoint, so each backward is the other.
# ---------------------------------------------------------------------------

def stream_expand(x, scale=1.0, n=4, dt=F64):
    """H[b,s,k,:] = scale * x[b,s,:] for k < n."""
    x = _a(x, dt)
    return np.repeat((dt(scale) * x)[:, :, None, :], n, axis=2)


def stream_collapse(H, scale=1.0, dt=F64):
    """y[b,s,:] = scale * sum_k H[b,s,k,:]."""
    return dt(scale) * _a(H, dt).sum(axis=2)


def stream_expand_backward(dH, scale=1.0, dt=F64):
    return stream_collapse(dH, scale, dt)


def stream_collapse_backward(dy, scale=1.0, n=4, dt=F64):
    return stream_expand(dy, scale, n, dt)


# ---------------------------------------------------------------------------
# Mean-pool (module.py:123) and static / unfused weights (module.py:108-117,141-163)
# ---------------------------------------------------------------------------

def mean_pool(H, dt=F64):
    H = _a(H, dt)
    B, S, n, D = H.shape
    return H.mean(axis=1).reshape(B, n * D)


def static_weights(H_pre_base, H_post_base, H_res_base, B, iters=20, dt=F64):
    """(H_post, H_pre, H_res) broadcast over B; H_post = sigmoid (no x2),
    normalisation and Sinkhorn with eps 1e-8."""
    bq, bp, br = _a(H_pre_base, dt), _a(H_post_base, dt), _a(H_res_base, dt)
    H_post = np.broadcast_to(sigmoid(bp), (B, 4)).copy()
    sg = sigmoid(bq)
    H_pre = np.broadcast_to(sg / (sg.sum() + 1e-8), (B, 4)).copy()
    H_res = np.broadcast_to(sinkhorn(br, iters, 1e-8, dt), (B, 4, 4)).copy()
    return H_post, H_pre, H_res


def static_weights_backward(H_pre_base, H_post_base, H_res_base, gH_post, gH_pre, gH_res, iters=20, dt=F64):
    """Gradients w.r.t. (H_pre_base, H_post_base, H_res_base)."""
    bq, bp, br = _a(H_pre_base, dt), _a(H_post_base, dt), _a(H_res_base, dt)
    gp = _a(gH_post, dt).sum(axis=0)
    gq = _a(gH_pre, dt).sum(axis=0)
    gr = _a(gH_res, dt).sum(axis=0)
    sp = sigmoid(bp)
    g_post_base = gp * sp * (1 - sp)
    sq = sigmoid(bq)
    den = sq.sum() + 1e-8
    Hq = sq / den
    g_pre_base = (gq - (gq * Hq).sum()) / den * sq * (1 - sq)
    g_res_base = sinkhorn_backward(br, gr, iters, 1e-8, dt)
    return g_pre_base, g_post_base, g_res_base


def unfused_weights(x, W_pre, W_post, W_res, s_pre, s_post, s_res, H_pre_base, H_post_base, H_res_base,
                    iters=20, eps=1e-6, dt=F64):
    """(H_post, H_pre, H_res) of the use_fused_weights=False path from the mean x [B,K]."""
    x = _a(x, dt)
    B, K = x.shape
    rms = np.sqrt((x * x).mean(axis=-1, keepdims=True) + dt(eps))
    xn = x / rms
    zp = _a(H_post_base, dt) + (xn @ _a(W_post, dt).T) * _s(s_post, dt)
    zq = _a(H_pre_base, dt) + (xn @ _a(W_pre, dt).T) * _s(s_pre, dt)
    zr = _a(H_res_base, dt) + (xn @ _a(W_res, dt).T).reshape(B, 4, 4) * _s(s_res, dt)
    H_post = sigmoid(zp)
    sq = sigmoid(zq)
    H_pre = sq / (sq.sum(axis=-1, keepdims=True) + 1e-8)
    H_res = sinkhorn(zr, iters, 1e-8, dt)
    return H_post, H_pre, H_res


def unfused_weights_backward(x, W_pre, W_post, W_res, s_pre, s_post, s_res, H_pre_base, H_post_base,
                             H_res_base, gH_post, gH_pre, gH_res, iters=20, eps=1e-6, dt=F64):
    """Gradients as a dict: x, W_pre/W_post/W_res, scale_pre/post/res, H_pre/post/res_base."""
    x = _a(x, dt)
    B, K = x.shape
    Wq, Wp, Wr = _a(W_pre, dt), _a(W_post, dt), _a(W_res, dt)
    rms = np.sqrt((x * x).mean(axis=-1, keepdims=True) + dt(eps))
    xn = x / rms
    lp, lq, lr = xn @ Wp.T, xn @ Wq.T, xn @ Wr.T
    zp = _a(H_post_base, dt) + lp * _s(s_post, dt)
    zq = _a(H_pre_base, dt) + lq * _s(s_pre, dt)
    zr = _a(H_res_base, dt) + (lr * _s(s_res, dt)).reshape(B, 4, 4)
    sp = sigmoid(zp)
    g_zp = _a(gH_post, dt) * sp * (1 - sp)
    sq = sigmoid(zq)
    den = sq.sum(axis=-1, keepdims=True) + 1e-8
    Hq = sq / den
    gq = _a(gH_pre, dt)
    g_zq = (gq - (gq * Hq).sum(axis=-1, keepdims=True)) / den * sq * (1 - sq)
    g_zr = sinkhorn_backward(zr, _a(gH_res, dt), iters, 1e-8, dt).reshape(B, 16)
    out = {
        "H_post_base": g_zp.sum(axis=0),
        "H_pre_base": g_zq.sum(axis=0),
        "H_res_base": g_zr.sum(axis=0).reshape(4, 4),
        "scale_post": np.array([(g_zp * lp).sum()]),
        "scale_pre": np.array([(g_zq * lq).sum()]),
        "scale_res": np.array([(g_zr * lr).sum()]),
        "W_post": (g_zp * _s(s_post, dt)).T @ xn,
        "W_pre": (g_zq * _s(s_pre, dt)).T @ xn,
        "W_res": (g_zr * _s(s_res, dt)).T @ xn,
    }
    g_xn = (g_zp * _s(s_post, dt)) @ Wp + (g_zq * _s(s_pre, dt)) @ Wq + (g_zr * _s(s_res, dt)) @ Wr
    # xn = x / rms, rms = sqrt(mean(x^2) + eps)
    out["x"] = g_xn / rms - x * (g_xn * x).sum(axis=-1, keepdims=True) / (K * rms ** 3)
    return out


# ---------------------------------------------------------------------------
# Whole HyperConnection layer (module.py:103-182 == _torch_baseline.py:169-336)
# ---------------------------------------------------------------------------

def layer_forward(p, H, bo, dynamic=True, fused=True, iters=20, eps=1e-6, dt=F64):
    """branch_input, H_new and a cache for layer_backward.

    p: dict of parameters by their module names (numpy arrays).
    """
    H, bo = _a(H, dt), _a(bo, dt)
    B, S, n, D = H.shape
    cache = {"H": H, "bo": bo, "dynamic": dynamic, "fused": fused, "iters": iters, "eps": eps, "dt": dt}
    if not dynamic:
        H_post, H_pre, H_res = static_weights(p["H_pre_base"], p["H_post_base"], p["H_res_base"], B, iters, dt)
    else:
        x = mean_pool(H, dt)
        cache["x"] = x
        if fused:
            bias = np.concatenate([_a(p["H_pre_base"], dt), _a(p["H_post_base"], dt),
                                   _a(p["H_res_base"], dt).reshape(16)])
            cache["bias"] = bias
            H_pre, H_post, H_res = dynamic_weights(x, p["phi"], bias, float(np.ravel(p["alpha_pre"])[0]),
                                                   float(np.ravel(p["alpha_post"])[0]),
                                                   float(np.ravel(p["alpha_res"])[0]), iters, eps, dt)
        else:
            H_post, H_pre, H_res = unfused_weights(
                x, p["W_pre"], p["W_post"], p["W_res"], float(np.ravel(p["scale_pre"])[0]),
                float(np.ravel(p["scale_post"])[0]), float(np.ravel(p["scale_res"])[0]),
                p["H_pre_base"], p["H_post_base"], p["H_res_base"], iters, eps, dt)
    bi, hr = stream_mix(H, H_pre, H_res, dt)
    H_new = add_residual(hr, bo, H_post, dt)
    cache.update(H_pre=H_pre, H_post=H_post, H_res=H_res)
    return bi, H_new, cache


def layer_backward(p, cache, dH_new, d_bi):
    """Gradients of <dH_new, H_new> + <d_bi, branch_input> w.r.t. H, branch_output
    and every parameter (dict keyed like the module's named_parameters, plus
    "H" and "bo")."""
    dt = cache["dt"]
    H, bo = cache["H"], cache["bo"]
    B, S, n, D = H.shape
    iters, eps = cache["iters"], cache["eps"]
    _, d_bo, dH_post = add_residual_backward(dH_new, bo, cache["H_post"], dt)
    dH, dH_pre, dH_res = stream_mix_backward(d_bi, dH_new, H, cache["H_pre"], cache["H_res"], dt)
    g = {"bo": d_bo}
    if not cache["dynamic"]:
        gq, gp, gr = static_weights_backward(p["H_pre_base"], p["H_post_base"], p["H_res_base"], dH_post,
                                             dH_pre, dH_res, iters, dt)
        g.update(H_pre_base=gq, H_post_base=gp, H_res_base=gr)
        g["H"] = dH
        return g
    x = cache["x"]
    if cache["fused"]:
        gx, gphi, gbias, ga = dynamic_weights_backward(
            x, p["phi"], cache["bias"], float(np.ravel(p["alpha_pre"])[0]), float(np.ravel(p["alpha_post"])[0]),
            float(np.ravel(p["alpha_res"])[0]), dH_pre, dH_post, dH_res, iters, eps, dt)
        g.update(phi=gphi, H_pre_base=gbias[0:4], H_post_base=gbias[4:8], H_res_base=gbias[8:24].reshape(4, 4),
                 alpha_pre=np.array([ga[0]]), alpha_post=np.array([ga[1]]), alpha_res=np.array([ga[2]]))
    else:
        u = unfused_weights_backward(
            x, p["W_pre"], p["W_post"], p["W_res"], float(np.ravel(p["scale_pre"])[0]),
            float(np.ravel(p["scale_post"])[0]), float(np.ravel(p["scale_res"])[0]), p["H_pre_base"],
            p["H_post_base"], p["H_res_base"], dH_post, dH_pre, dH_res, iters, eps, dt)
        gx = u.pop("x")
        for k, v in u.items():
            g[k + (".weight" if k.startswith("W_") else "")] = v
    # mean-pool backward: dH[b,s,n,d] += gx[b, n*D + d] / S
    dH = dH + (gx.reshape(B, 1, n, D) / S)
    g["H"] = dH
    return g
