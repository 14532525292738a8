"""Tensors past 2^31 elements (4 GiB and more of bf16).

The reference indexes its Triton kernels from 64-bit program ids times strides
(src/mhc/_kernels.py:643,678,741; _backward.py:562,612), so a caller may pass tensors of any
size.  Here every launch reaches its rows and batches from 64-bit base offsets (row r at r * K,
batch b at b * S * 4 * D) and indexes inside per-workgroup buffer spans kept under 2^31 bytes.
These tests put data past 2^31 elements and check it, bit for bit, against runs over a window of
the same rows or batches that stays below that size and uses the same launch plan, so that the
per-row and per-batch arithmetic is the same instruction for instruction (the layer step's dH to
one bf16 rounding, for the reason its test gives):

* ``fused_dynamic_weights`` forward and backward at R * K = 2.16e9 (bf16 rows, MFMA kernels);
* ``fused_stream_mix`` / ``fused_add_residual`` forward and backward, and a dynamic
  ``HyperConnection`` step, on H of 65 x 2048 x 4 x 4096 = 2.18e9 elements: batch 32 starts at
  2^31 bytes, batch 64 at 2^31 elements.

The inputs past the boundary differ from those 2^31 elements (or bytes) before them, so that an
offset that wrapped would read other values.  Sums over the whole tensor (grad_phi and the layer's
parameter gradients) are checked against the sums of the windows' results.
"""

import pytest
import torch

from helpers import rel_err, to_np

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _same(what, got, want):
    if torch.equal(got, want):
        print(f"{what}: same bits", flush=True)
        return
    diff = (got.float() - want.float()).abs().max().item()
    raise AssertionError(f"{what}: differs, max |diff| {diff:.3e}")


def _close(what, got, want, tol):
    e = rel_err(to_np(got), to_np(want))
    print(f"{what}: {e:.2e}", flush=True)
    assert e < tol, (what, e)


def test_dynamic_weights_rows_past_2p31_elements():
    """R = 131,936 rows of K = 16384 bf16: 992 distinct rows repeated 133 times.  Row r and row
    r - 2^31 / K = r - 131,072 hold different rows (131,072 % 992 = 128).  992 is a multiple of
    the 32-row tile, so that each row sits at the same tile position in both runs."""
    from mhc import _backward as KB
    from mhc import _kernels as KF

    R0, N, K = 992, 133, 16384
    R = R0 * N
    assert R * K > 2 ** 31 and (2 ** 31 // K) % R0 != 0
    g = torch.Generator(device=DEV).manual_seed(21)
    x0 = (torch.randn((R0, K), generator=g, device=DEV) / 64).to(torch.bfloat16)
    phi = torch.randn((K, 24), generator=g, device=DEV) * 0.02
    bias = torch.randn(24, generator=g, device=DEV) * 0.1
    al = [torch.tensor([v], device=DEV) for v in (0.1, 0.2, 0.3)]
    gw0 = [torch.randn(s, generator=g, device=DEV) for s in ((R0, 4), (R0, 4), (R0, 4, 4))]

    print(f"dynamic weights R={R} K={K} bf16 ({R * K} elements)", flush=True)
    f0 = KF.fused_dynamic_weights_forward(x0, phi, bias, *al, return_aux=True)
    b0 = KB.fused_dynamic_weights_backward(x0, phi, bias, al, f0[3], f0[0], *gw0, 20, 1e-6)
    x = x0.repeat(N, 1)
    gw = [t.repeat(N, *([1] * (t.dim() - 1))) for t in gw0]
    f = KF.fused_dynamic_weights_forward(x, phi, bias, *al, return_aux=True)
    b = KB.fused_dynamic_weights_backward(x, phi, bias, al, f[3], f[0], *gw, 20, 1e-6)
    torch.cuda.synchronize()
    for name, big, small in zip(("H_pre", "H_post", "H_res", "aux", "grad_x"), (*f, b[0]), (*f0, b0[0])):
        _same(f"{name} (every block of {R0} rows)", big, small.repeat(N, *([1] * (small.dim() - 1))))
    # the parameter gradients sum over all rows: N times the window's, up to fp32 summation
    # order (grad_phi accumulates 33k rows per chunk in one MFMA chain: about 1e-5 of its size)
    for name, big, small in zip(("grad_phi", "grad_bias", "grad_alpha"), b[1:], b0[1:]):
        _close(name, big, small * N, 1e-4)


def _stream_inputs(B, S, D, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    mk = lambda *shape: torch.randn(shape, generator=g, device=DEV, dtype=torch.bfloat16)  # noqa: E731
    H, bo, dHn, dbi = mk(B, S, 4, D), mk(B, S, D), mk(B, S, 4, D), mk(B, S, D)
    pre = torch.softmax(torch.randn((B, 4), generator=g, device=DEV), -1)
    res = torch.rand((B, 4, 4), generator=g, device=DEV)
    post = 2 * torch.rand((B, 4), generator=g, device=DEV)
    return H, bo, dHn, dbi, pre, res, post


B, S, D = 65, 2048, 4096
WINDOWS = [slice(0, 48), slice(17, 65)]  # each below 2^31 elements; together every batch


def test_stream_ops_past_2p31_elements():
    """fused_stream_mix and fused_add_residual, forward and backward, on 65 batches against
    windows of 48 batches (per-element outputs and per-batch reductions over the same tiles)."""
    from mhc import _backward as KB
    from mhc import _kernels as KF

    assert B * S * 4 * D > 2 ** 31
    H, bo, dHn, dbi, pre, res, post = _stream_inputs(B, S, D, 22)
    print(f"stream ops B={B} S={S} D={D} bf16 ({B * S * 4 * D} elements)", flush=True)

    def run(sl):
        bi, hr = KF.stream_mix_forward(H[sl], pre[sl], res[sl])
        dH, dpre, dres = KB.stream_mix_backward(dbi[sl], dHn[sl], H[sl], pre[sl], res[sl])
        Hn = KF.add_residual_forward(hr, bo[sl], post[sl])
        _, dbo, dpost = KB.add_residual_backward(dHn[sl], bo[sl], post[sl])
        return {"branch_input": bi, "H_residual": hr, "dH": dH, "dH_pre": dpre, "dH_res": dres, "H_new": Hn,
                "d_branch_output": dbo, "dH_post": dpost}

    big = run(slice(None))
    torch.cuda.synchronize()
    for sl in WINDOWS:
        win = run(sl)
        for k, v in win.items():
            _same(f"{k} batches {sl.start}..{sl.stop - 1}", big[k][sl], v)
        del win


LAYER_WINDOWS = [slice(0, 64), slice(1, 65)]  # 2^31 elements each: indices below 2^31


def test_layer_step_past_2p31_elements():
    """A dynamic HyperConnection step (mean-pool projection, weights, mix, closure and every
    gradient, the weights backward on the MFMA kernel) on 65 batches against windows of 64.  The
    forward (the mean-pool's S split is the same for 64 and 65 batches at this shape) and
    d_branch_output match bit for bit.  dH is the exception by design: pass B
    spreads each batch's dH_pre / dH_res sums over a number of workgroups that depends on the
    batch count, so the weight gradients, and with them the mean-pool term grad_x / S inside dH,
    differ in their last fp32 bits; a few dH elements then round to the neighbouring bf16 value."""
    import mhc

    assert B * S * 4 * D > 2 ** 31
    torch.manual_seed(23)
    hc = mhc.HyperConnection(D, dynamic=True, layer_idx=1).to(DEV)
    with torch.no_grad():
        hc.phi.normal_(0.0, 0.02)
    H, bo, dHn, dbi, *_ = _stream_inputs(B, S, D, 24)
    print(f"layer step B={B} S={S} D={D} bf16 ({B * S * 4 * D} elements)", flush=True)

    def run(sl):
        Hl = H[sl].clone().requires_grad_(True)
        bol = bo[sl].clone().requires_grad_(True)
        hc.zero_grad(set_to_none=True)
        bi, add = hc(Hl)
        Hn = add(bol)
        torch.autograd.backward([Hn, bi], [dHn[sl], dbi[sl]])
        out = {"branch_input": bi.detach(), "H_new": Hn.detach(), "dH": Hl.grad, "d_branch_output": bol.grad}
        return out, {n: p.grad.clone() for n, p in hc.named_parameters()}

    big, big_p = run(slice(None))
    torch.cuda.synchronize()
    for sl in LAYER_WINDOWS:
        win, _ = run(sl)
        for k, v in win.items():
            what = f"{k} batches {sl.start}..{sl.stop - 1}"
            if k != "dH":
                _same(what, big[k][sl], v)
                continue
            got = big[k][sl]
            flips = (got != v).float().mean().item()
            # one bf16 step of the larger of the two values (2^(e - 7) for magnitudes in
            # [2^e, 2^(e+1))), plus 1e-4 of the tensor's largest value (the fp32 gradient
            # tolerance) for values near zero, whose steps are finer than the fp32 differences
            a, w = got.float(), v.float()
            m = torch.maximum(a.abs(), w.abs())
            step = torch.exp2(torch.floor(torch.log2(m.clamp_min(1e-30))) - 7)
            over = ((a - w).abs() > step + 1e-4 * w.abs().max()).sum().item()
            print(f"{what}: {flips:.2e} of the elements differ, {over} by more than one bf16 step",
                  flush=True)
            assert flips < 1e-3 and over == 0, (what, flips, over)
            del a, w, m, step
        del win
    # parameter gradients: the sum over all batches, from two windows that split them
    _, p0 = run(slice(0, 64))
    _, p1 = run(slice(64, 65))
    for n, v in big_p.items():
        _close(f"grad {n}", v, p0[n] + p1[n], 1e-5)
