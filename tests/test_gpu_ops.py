"""GPU parity of the low-level ops (mhc.sinkhorn_knopp, fused_stream_mix,
fused_add_residual, fused_dynamic_weights) against the float64 oracle.

Tolerances (normwise relative error, max|y - y_ref| / max|y_ref|):
  fp32 forward 1e-5, fp32 gradients 1e-4, outputs from bf16/fp16 inputs 2e-2
(the oracle is fed the same bf16/fp16 values, upcast).
"""

import numpy as np
import pytest
import torch

from helpers import rel_err, to_np
from oracle import mhc_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}
GTOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def gen(seed=0):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def randn(shape, g, dtype=torch.float32, scale=1.0):
    return (torch.randn(shape, generator=g, dtype=torch.float32) * scale).to(dtype).to(DEV)


# --------------------------------------------------------------------------- Sinkhorn

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_sinkhorn_forward(dtype):
    import mhc

    g = gen(0)
    M = randn((1000, 4, 4), g, dtype)
    P = mhc.sinkhorn_knopp(M, 20)
    assert P.dtype == dtype and P.shape == M.shape
    assert rel_err(to_np(P), O.sinkhorn(to_np(M), 20, 1e-8)) < TOL[dtype]


@pytest.mark.parametrize("iters", [0, 1, 7, 20, 21, 33, 64, 65])
def test_sinkhorn_forward_backward_iters(iters):
    """Up to 20 rounds the backward keeps every round's scaling vectors in registers; from 21 to
    64 it recomputes them segment by segment (16 rounds each) from checkpoints; beyond that it
    recomputes explicit states from checkpoints.  Each is held to the oracle, and the 16-byte
    load path to the element-wise one."""
    import mhc

    g = gen(1)
    M = randn((300, 4, 4), g)
    M[0, 0, 0] = 0.0  # exercise sgn(0) = 0
    M[7, 2, 1] = 0.0
    dP = randn((300, 4, 4), g)
    Ml = M.clone().requires_grad_(True)
    P = mhc.sinkhorn_knopp(Ml, iters, 1e-8)
    P.backward(dP)
    assert rel_err(to_np(P), O.sinkhorn(to_np(M), iters, 1e-8)) < 1e-5
    ref = O.sinkhorn_backward(to_np(M), to_np(dP), iters, 1e-8)
    assert rel_err(to_np(Ml.grad), ref) < 1e-4
    assert Ml.grad[0, 0, 0].item() == 0.0 and Ml.grad[7, 2, 1].item() == 0.0
    # the same matrices at an offset of one element: the element-wise load path
    flat = torch.cat([torch.zeros(1, device=DEV), M.reshape(-1)]).requires_grad_(True)
    Mu = flat[1:].view(300, 4, 4)
    assert Mu.data_ptr() % 16 != 0
    mhc.sinkhorn_knopp(Mu, iters, 1e-8).backward(dP)
    gu = flat.grad[1:].view(300, 4, 4)
    assert rel_err(to_np(gu), to_np(Ml.grad)) < 1e-5


def test_sinkhorn_config2_column_sums_and_oracle():
    """Config 2: 2^20 log-normal fp32 matrices, 20 iterations, N(0,1) upstream gradient."""
    import mhc

    g = gen(0)
    n = 1 << 20
    M = torch.exp(torch.randn((n, 4, 4), generator=g)).to(DEV)
    dP = torch.randn((n, 4, 4), generator=g).to(DEV)
    Ml = M.clone().requires_grad_(True)
    P = mhc.sinkhorn_knopp(Ml, 20)
    P.backward(dP)
    Pn = to_np(P)
    # columns: last step of every round, so |colsum - 1| <= 1e-5 for every matrix
    assert np.abs(Pn.sum(-2) - 1).max() < 1e-5
    Mn = to_np(M)
    ref = O.sinkhorn(Mn, 20, 1e-8)
    assert rel_err(Pn, ref) < 1e-5
    # rows: the reference algorithm itself leaves some rows unconverged at 20
    # iterations; row sums must match the oracle's, not 1
    assert np.abs(Pn.sum(-1) - ref.sum(-1)).max() < 1e-5
    sub = slice(0, 1 << 16)
    gref = O.sinkhorn_backward(Mn[sub], to_np(dP)[sub], 20, 1e-8)
    assert rel_err(to_np(Ml.grad)[sub], gref) < 1e-4


def test_sinkhorn_edge_cases():
    import mhc

    empty = torch.empty(0, 4, 4, device=DEV)
    assert mhc.sinkhorn_knopp(empty).shape == (0, 4, 4)
    g = gen(2)
    base = randn((65, 4, 4), g)
    # unaligned view (offset of one element) takes the scalar path
    flat = torch.cat([torch.zeros(1, device=DEV), base.reshape(-1)])
    M = flat[1:].view(65, 4, 4)
    assert M.data_ptr() % 16 != 0
    P = mhc.sinkhorn_knopp(M)
    assert rel_err(to_np(P), O.sinkhorn(to_np(base), 20, 1e-8)) < 1e-5
    # non-contiguous input
    Mt = base.transpose(1, 2)
    P = mhc.sinkhorn_knopp(Mt)
    assert rel_err(to_np(P), O.sinkhorn(to_np(Mt), 20, 1e-8)) < 1e-5
    with pytest.raises(AssertionError):
        mhc.sinkhorn_knopp(torch.zeros(3, 4, 5, device=DEV))


# --------------------------------------------------------------------------- stream mix

# (2, 33, 136): several tiles with a partial last one on the 16-byte vector path for every dtype
MIX_SHAPES = [(2, 64, 256), (3, 7, 100), (1, 5, 130), (2, 1, 8), (2, 33, 136)]


def _weights(B, g):
    H_pre = torch.softmax(torch.randn((B, 4), generator=g), -1).to(DEV)
    H_res = torch.tensor(O.sinkhorn(torch.randn((B, 4, 4), generator=g).numpy(), 20, 1e-8),
                         dtype=torch.float32).to(DEV)
    return H_pre, H_res


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", MIX_SHAPES)
def test_stream_mix_forward_backward(dtype, shape):
    import mhc

    B, S, D = shape
    g = gen(3)
    H = randn((B, S, 4, D), g, dtype)
    H_pre, H_res = _weights(B, g)
    d_bi = randn((B, S, D), g, dtype)
    d_hr = randn((B, S, 4, D), g, dtype)
    Hl, pl, rl = (t.clone().requires_grad_(True) for t in (H, H_pre, H_res))
    bi, hr = mhc.fused_stream_mix(Hl, pl, rl)
    assert bi.dtype == dtype and hr.dtype == dtype
    torch.autograd.backward([bi, hr], [d_bi, d_hr])
    obi, ohr = O.stream_mix(to_np(H), to_np(H_pre), to_np(H_res))
    assert rel_err(to_np(bi), obi) < TOL[dtype]
    assert rel_err(to_np(hr), ohr) < TOL[dtype]
    dH, dpre, dres = O.stream_mix_backward(to_np(d_bi), to_np(d_hr), to_np(H), to_np(H_pre), to_np(H_res))
    assert rel_err(to_np(Hl.grad), dH) < GTOL[dtype]
    assert pl.grad.dtype == torch.float32 and rl.grad.dtype == torch.float32
    assert rel_err(to_np(pl.grad), dpre) < 1e-4
    assert rel_err(to_np(rl.grad), dres) < 1e-4


# --------------------------------------------------------------------------- add residual

@pytest.mark.parametrize("dtype,bo_dtype", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                            (torch.float16, torch.float16), (torch.bfloat16, torch.float32),
                                            (torch.float32, torch.bfloat16)])
@pytest.mark.parametrize("shape", MIX_SHAPES)
def test_add_residual_forward_backward(dtype, bo_dtype, shape):
    import mhc

    B, S, D = shape
    g = gen(4)
    hr = randn((B, S, 4, D), g, dtype)
    bo = randn((B, S, D), g, bo_dtype)
    H_post = torch.sigmoid(torch.randn((B, 4), generator=g)).to(DEV) * 2
    dHn = randn((B, S, 4, D), g, dtype)
    hl, bl, pl = (t.clone().requires_grad_(True) for t in (hr, bo, H_post))
    Hn = mhc.fused_add_residual(hl, bl, pl)
    assert Hn.dtype == dtype
    Hn.backward(dHn)
    tol = max(TOL[dtype], TOL[bo_dtype])
    assert rel_err(to_np(Hn), O.add_residual(to_np(hr), to_np(bo), to_np(H_post))) < tol
    _, dbo, dpost = O.add_residual_backward(to_np(dHn), to_np(bo), to_np(H_post))
    assert torch.equal(hl.grad, dHn)
    assert bl.grad.dtype == bo_dtype
    assert rel_err(to_np(bl.grad), dbo) < max(GTOL[dtype], GTOL[bo_dtype])
    assert rel_err(to_np(pl.grad), dpost) < 1e-4


# --------------------------------------------------------------------------- dynamic weights

@pytest.mark.parametrize("R,K,xdtype", [(4, 16384, torch.float32), (1, 28672, torch.float32),
                                        (37, 1000, torch.float32), (4, 16384, torch.bfloat16),
                                        (300, 2048, torch.float16),
                                        # bf16 rows in bulk take the MFMA projection (ragged last tile)
                                        (1000, 4096, torch.bfloat16), (4096, 16384, torch.bfloat16),
                                        (64, 1040, torch.bfloat16),
                                        # a last K chunk that ends inside a wave's slice, a one-row tile
                                        (257, 3008, torch.bfloat16),
                                        # one 16-k step (seven of the eight waves' slices past K)
                                        (65, 16, torch.bfloat16),
                                        # K % 16 = 8: the VALU projection forward, the MFMA backward
                                        (100, 1000, torch.bfloat16),
                                        # MFMA backward row chunks of 188 rows (two whole 64-row
                                        # blocks and a partial one), eight chunk partials
                                        (1500, 8192, torch.bfloat16),
                                        # MFMA forward with rows in bulk: 9 chunks, the last one step
                                        # long (seven of its eight waves' slices past K), a last row
                                        # range of 11 tiles (an odd count, the last one partial)
                                        (21845, 8208, torch.bfloat16),
                                        # fp16 rows on the MFMA kernels (x split into two bf16 parts)
                                        (1000, 4096, torch.float16), (257, 3008, torch.float16),
                                        (4096, 16384, torch.float16), (21845, 8208, torch.float16),
                                        # fp32 rows on the MFMA kernels (x in three bf16 parts
                                        # forward, 512-k chunks): a last chunk of 28 steps (the last
                                        # wave's slice past K), one step, a one-step last chunk;
                                        # backward column blocks of 16 and 192 columns
                                        (1000, 4096, torch.float32), (257, 3008, torch.float32),
                                        (65, 16, torch.float32), (21845, 8208, torch.float32),
                                        (4096, 16384, torch.float32),
                                        # K % 16 = 8: the VALU projection forward, the MFMA backward
                                        # with a last column block of 232 columns
                                        (100, 1000, torch.float32), (100, 1000, torch.float16)])
def test_dynamic_weights_forward_backward(R, K, xdtype):
    import mhc

    g = gen(5)
    # x as a sequence mean of unit normals (std ~ 1/64), phi ~ N(0, 0.02)
    x = randn((R, K), g, xdtype, scale=1 / 64)
    phi = randn((K, 24), g, scale=0.02)
    bias = torch.cat([torch.tensor([1.0, 0, 0, 0]), torch.ones(4), torch.eye(4).flatten()]).to(DEV)
    bias = bias + randn((24,), g, scale=0.1)
    alphas = [torch.tensor([v], device=DEV) for v in (0.1, 0.2, 0.3)]
    gp, gq, gr = randn((R, 4), g), randn((R, 4), g), randn((R, 4, 4), g)
    leaves = [t.clone().requires_grad_(True) for t in (x, phi, bias, *alphas)]
    H_pre, H_post, H_res = mhc.fused_dynamic_weights(*leaves, 20, 1e-6)
    assert H_pre.dtype == H_post.dtype == H_res.dtype == torch.float32
    torch.autograd.backward([H_pre, H_post, H_res], [gp, gq, gr])
    args = [to_np(x), to_np(phi), to_np(bias)] + [a.item() for a in alphas]
    oq, op, orr = O.dynamic_weights(*args, 20, 1e-6)
    assert rel_err(to_np(H_pre), oq) < 1e-5
    assert rel_err(to_np(H_post), op) < 1e-5
    # The 20-round Sinkhorn amplifies the projection's fp32 rounding about 10x:
    # at R = 4096, K = 16384 the oracle itself run in fp32 is 4e-6 off its fp64
    # result for H_res.  Outputs from bf16/fp16 x may be 2e-2 off; hold them to 5e-5.
    assert rel_err(to_np(H_res), orr) < (1e-5 if xdtype == torch.float32 else 5e-5)
    gx, gphi, gbias, ga = O.dynamic_weights_backward(*args, to_np(gp), to_np(gq), to_np(gr), 20, 1e-6)
    print(f"dynamic weights R={R} K={K} {xdtype}: H_res {rel_err(to_np(H_res), orr):.2e} "
          f"grad_x {rel_err(to_np(leaves[0].grad), gx):.2e} grad_phi {rel_err(to_np(leaves[1].grad), gphi):.2e}",
          flush=True)
    assert leaves[0].grad.dtype == xdtype
    assert rel_err(to_np(leaves[0].grad), gx) < GTOL[xdtype]
    if xdtype == torch.bfloat16:
        # grad_x is formed in fp32 (on MFMA from split bf16 operands for R >= 64) and rounded
        # once to bf16: within half a bf16 ulp, 2^-9, of the largest element.
        assert rel_err(to_np(leaves[0].grad), gx) < 4e-3
    if xdtype == torch.float16:
        # likewise rounded once to fp16: half an fp16 ulp is 2^-12 of the largest element
        assert rel_err(to_np(leaves[0].grad), gx) < 5e-4
    assert rel_err(to_np(leaves[1].grad), gphi) < 1e-4
    assert rel_err(to_np(leaves[2].grad), gbias) < 1e-4
    assert rel_err(np.array([a.grad.item() for a in leaves[3:]]), np.array(ga)) < 1e-4


@pytest.mark.parametrize("R,K,xdtype", [(1000, 4096, torch.bfloat16), (257, 3008, torch.bfloat16),
                                        (21845, 8208, torch.bfloat16), (1000, 4096, torch.float16),
                                        (1000, 4096, torch.float32)])
def test_dynamic_weights_mfma_paths_are_deterministic(R, K, xdtype):
    """The MFMA projection adds its waves' tile results and the K chunks in a fixed order, and the
    backward's grad_phi / bias partials likewise: two calls give the same bits."""
    import mhc

    g = gen(8)
    x = randn((R, K), g, xdtype, scale=1 / 64)
    phi = randn((K, 24), g, scale=0.02)
    bias = randn((24,), g, scale=0.1)
    alphas = [torch.tensor([v], device=DEV) for v in (0.1, 0.2, 0.3)]
    gouts = [randn((R, 4), g), randn((R, 4), g), randn((R, 4, 4), g)]
    runs = []
    for _ in range(2):
        leaves = [t.clone().requires_grad_(True) for t in (x, phi, bias, *alphas)]
        outs = mhc.fused_dynamic_weights(*leaves, 20, 1e-6)
        torch.autograd.backward(list(outs), gouts)
        runs.append([o.detach() for o in outs] + [t.grad for t in leaves])
    for a, b in zip(*runs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("xdtype", [torch.float16, torch.bfloat16, torch.float32])
def test_dynamic_weights_projection_over_a_wide_phi_range(xdtype):
    """The MFMA projection (aux[:, :24] = x phi) per column, against float64, for phi columns
    far outside fp16's range (1e5), far below it (1e-9, and for fp16 x 1e-36), all zero, and
    N(0, 0.02): the fp16 path scales each column by a power of two before splitting it into
    fp16 parts, the bf16 / fp32 paths split it into bf16 parts (fp32's exponent range)."""
    from mhc import _kernels as K_

    R, K = 256, 2048
    g = gen(11)
    x = randn((R, K), g, xdtype, scale=1 / 64)
    phi = randn((K, 24), g, scale=0.02)
    phi[:, 0] *= 5e6
    phi[:, 1] *= 5e-8
    phi[:, 2] = 0.0
    phi[::7, 3] *= 1e4  # one column with a few large entries among ordinary ones
    if xdtype == torch.float16:
        phi[:, 4] *= 5e-35  # largest entry near 2^-118: the scale is held at 2^126
    bias = randn((24,), g, scale=0.1)
    alphas = [torch.tensor([v], device=DEV) for v in (0.1, 0.2, 0.3)]
    *_, aux = K_.fused_dynamic_weights_forward(x, phi, bias, *alphas, return_aux=True)
    raw = to_np(x) @ to_np(phi)
    got = to_np(aux[:, :24])
    errs = [rel_err(got[:, j], raw[:, j]) for j in range(24) if j != 2]
    print(f"{xdtype}: worst column error {max(errs):.2e}", flush=True)
    assert max(errs) < 1e-5
    assert np.all(got[:, 2] == 0.0)
    ss = (to_np(x) ** 2).sum(axis=1)
    assert rel_err(1.0 / to_np(aux[:, 24]) ** 2, ss / K + 1e-6) < 1e-5


def test_dynamic_weights_default_init_sgn_zero():
    """phi = 0 with the module's default bias: scaled_res has 12 exact zeros,
    whose gradient follows torch (sgn(0) = 0)."""
    import mhc

    R, K = 4, 2048
    g = gen(6)
    x = randn((R, K), g, scale=1 / 64)
    phi = torch.zeros(K, 24, device=DEV)
    bias = torch.cat([torch.tensor([1.0, 0, 0, 0]), torch.ones(4), torch.eye(4).flatten()]).to(DEV)
    alphas = [torch.tensor([0.1], device=DEV) for _ in range(3)]
    leaves = [t.clone().requires_grad_(True) for t in (x, phi, bias, *alphas)]
    outs = mhc.fused_dynamic_weights(*leaves)
    gs = [randn(o.shape, g) for o in outs]
    torch.autograd.backward(list(outs), gs)
    args = [to_np(x), to_np(phi), to_np(bias)] + [0.1, 0.1, 0.1]
    gx, gphi, gbias, ga = O.dynamic_weights_backward(*args, *[to_np(t) for t in gs], 20, 1e-6)
    assert torch.count_nonzero(leaves[0].grad).item() == 0  # grad_x == 0 exactly
    assert rel_err(to_np(leaves[1].grad), gphi) < 1e-4
    assert rel_err(to_np(leaves[2].grad), gbias) < 1e-4
    zero_res = (np.eye(4).reshape(16) == 0)
    assert np.all(to_np(leaves[2].grad)[8:24][zero_res] == 0.0)


def test_mean_pool_matches_oracle():
    from mhc._kernels import mean_pool

    g = gen(7)
    # S <= 8, or up to 64 in one S chunk: the single-launch form (colsum_direct_vec_kernel, or
    # colsum_direct_kernel for unaligned rows); longer or split: column sums + reduce
    for dtype, shape in [(torch.float32, (2, 128, 4, 512)), (torch.bfloat16, (3, 77, 4, 100)),
                         (torch.float16, (1, 300, 4, 64)), (torch.bfloat16, (5, 1, 4, 1024)),
                         (torch.float32, (2, 8, 4, 96)), (torch.float16, (3, 3, 4, 50)),
                         (torch.bfloat16, (200, 20, 4, 1024)), (torch.float32, (400, 64, 4, 128))]:
        H = randn(shape, g, dtype)
        x = mean_pool(H)
        assert x.dtype == torch.float32
        assert rel_err(to_np(x), O.mean_pool(to_np(H))) < 1e-5


# --------------------------------------------------------------------------- empty inputs

@pytest.mark.parametrize("B,S", [(0, 8), (2, 0)])
def test_stream_ops_empty(B, S):
    """Zero-size batch or sequence: empty outputs, zero weight gradients, no launch errors."""
    import mhc

    D = 16
    H = torch.zeros((B, S, 4, D), device=DEV, requires_grad=True)
    pre = torch.full((B, 4), 0.25, device=DEV, requires_grad=True)
    res = torch.full((B, 4, 4), 0.25, device=DEV, requires_grad=True)
    bi, hr = mhc.fused_stream_mix(H, pre, res)
    assert bi.shape == (B, S, D) and hr.shape == (B, S, 4, D)
    bo = torch.zeros((B, S, D), device=DEV, requires_grad=True)
    post = torch.ones((B, 4), device=DEV, requires_grad=True)
    H_new = mhc.fused_add_residual(hr, bo, post)
    (H_new.sum() + bi.sum()).backward()
    torch.cuda.synchronize()
    assert H.grad.shape == H.shape and float(pre.grad.abs().sum()) == 0.0
    assert float(res.grad.abs().sum()) == 0.0 and float(post.grad.abs().sum()) == 0.0


def test_dynamic_weights_zero_rows():
    import mhc

    K = 32
    x = torch.zeros((0, K), device=DEV, requires_grad=True)
    phi = torch.randn((K, 24), device=DEV, requires_grad=True)
    bias = torch.randn(24, device=DEV, requires_grad=True)
    al = [torch.tensor([0.1], device=DEV, requires_grad=True) for _ in range(3)]
    H_pre, H_post, H_res = mhc.fused_dynamic_weights(x, phi, bias, *al)
    assert H_pre.shape == (0, 4) and H_res.shape == (0, 4, 4)
    (H_pre.sum() + H_post.sum() + H_res.sum()).backward()
    torch.cuda.synchronize()
    assert float(phi.grad.abs().sum()) == 0.0 and float(bias.grad.abs().sum()) == 0.0
