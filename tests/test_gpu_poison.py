"""Every output and workspace entry is written before it is read.

The reference's launchers allocate outputs and per-call workspaces with torch.empty
(reference src/mhc/_kernels.py:640-641, _backward.py:560,609-610), and so do this
build's: include/mhc_abi.h documents that each entry point overwrites every entry it
reads.  Here each op, the layer launchers and the three HyperConnection kinds run twice:
once plainly, once with torch.empty, torch.empty_like and Tensor.new_empty patched to fill
floating-point tensors with NaN and byte tensors (the workspaces) with 0xFF.  A kernel that
read an entry it had not written would carry the NaN (or the garbage float 0xFFFFFFFF) into
its outputs, so every result must come out bit-identical.
"""

import contextlib

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


@contextlib.contextmanager
def poisoned_allocations():
    empty, empty_like, new_empty = torch.empty, torch.empty_like, torch.Tensor.new_empty

    def fill(t):
        if t.is_floating_point():
            t.fill_(float("nan"))
        elif t.dtype == torch.uint8:
            t.fill_(0xFF)
        return t

    torch.empty = lambda *a, **k: fill(empty(*a, **k))
    torch.empty_like = lambda *a, **k: fill(empty_like(*a, **k))
    torch.Tensor.new_empty = lambda self, *a, **k: fill(new_empty(self, *a, **k))
    try:
        yield
    finally:
        torch.empty, torch.empty_like, torch.Tensor.new_empty = empty, empty_like, new_empty


def _same(ref, got):
    assert ref.keys() == got.keys()
    for k in ref:
        a, b = ref[k], got[k]
        if a is None or b is None:
            assert a is None and b is None, k
            continue
        assert a.dtype == b.dtype and a.shape == b.shape, k
        assert torch.equal(a, b) or (a.isnan().all() and b.isnan().all()), (k, int((a != b).sum()))


def _twice(run):
    ref = run()
    torch.cuda.synchronize()
    with poisoned_allocations():
        got = run()
        torch.cuda.synchronize()
    _same(ref, got)


def _rand(g, *shape, dtype=torch.float32, scale=1.0):
    return (torch.randn(shape, generator=g, device=DEV) * scale).to(dtype)


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 256), (torch.float32, 72), (torch.float16, 100)])
def test_public_ops_overwrite_what_they_read(dtype, D):
    import mhc

    g = torch.Generator(device=DEV).manual_seed(0)
    B, S = 3, 40
    H = _rand(g, B, S, 4, D, dtype=dtype)
    pre = torch.rand((B, 4), generator=g, device=DEV)
    res = torch.rand((B, 4, 4), generator=g, device=DEV)
    post = torch.rand((B, 4), generator=g, device=DEV)
    bo = _rand(g, B, S, D, dtype=dtype)
    dbi, dhr = _rand(g, B, S, D, dtype=dtype), _rand(g, B, S, 4, D, dtype=dtype)
    M = _rand(g, 70, 4, 4).exp()
    dP = _rand(g, 70, 4, 4)
    x = _rand(g, B, 4 * D, dtype=dtype)
    phi = _rand(g, 4 * D, 24, scale=0.02)
    bias = _rand(g, 24)
    al = [torch.tensor([0.1 * (i + 1)], device=DEV) for i in range(3)]

    def run():
        out = {}
        leaves = [t.clone().requires_grad_(True) for t in (M, H, pre, res, bo, post, x, phi, bias, *al)]
        Ml, Hl, pl, rl, bol, ql, xl, phil, bl, a0, a1, a2 = leaves
        P = mhc.sinkhorn_knopp(Ml, 20)
        bi, hr = mhc.fused_stream_mix(Hl, pl, rl)
        Hn = mhc.fused_add_residual(hr, bol, ql)
        wp, wq, wr = mhc.fused_dynamic_weights(xl, phil, bl, a0, a1, a2)
        y = mhc.streams.collapse_streams(mhc.streams.expand_streams(bol), reduction="mean")
        out.update(P=P, bi=bi, hr=hr, Hn=Hn, wp=wp, wq=wq, wr=wr, y=y)
        torch.autograd.backward([P, bi, Hn, wp, wr, y],
                                [dP, dbi, dhr, wp.detach() * 0 + 1, dP[:B], bo])
        for name, t in zip(("M", "H", "pre", "res", "bo", "post", "x", "phi", "bias", "a0", "a1", "a2"), leaves):
            out["d" + name] = t.grad
        out["pool"] = mhc._kernels.mean_pool(H)
        return out

    _twice(run)


def test_mfma_dynamic_weights_overwrite_what_they_read():
    """bf16 rows in bulk: the MFMA projection, its split-K records and the MFMA backward's
    row-chunk partials, with a ragged last tile."""
    import mhc

    g = torch.Generator(device=DEV).manual_seed(1)
    R, K = 257, 1040
    x = _rand(g, R, K, dtype=torch.bfloat16)
    phi = _rand(g, K, 24, scale=0.02)
    bias = _rand(g, 24)
    al = [torch.tensor([0.2], device=DEV) for _ in range(3)]
    gp, gq, gr = _rand(g, R, 4), _rand(g, R, 4), _rand(g, R, 4, 4)

    def run():
        xl, pl, bl = (t.clone().requires_grad_(True) for t in (x, phi, bias))
        wp, wq, wr = mhc.fused_dynamic_weights(xl, pl, bl, *al)
        torch.autograd.backward([wp, wq, wr], [gp, gq, gr])
        return {"wp": wp, "wq": wq, "wr": wr, "dx": xl.grad, "dphi": pl.grad, "dbias": bl.grad}

    _twice(run)


@pytest.mark.parametrize("kind", ["dynamic", "static", "unfused"])
@pytest.mark.parametrize("closure", ["used", "called_no_grad", "never_called"])
@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 256), (torch.float32, 100)])
def test_layer_overwrites_what_it_reads(kind, closure, dtype, D):
    """HyperConnection forward + backward, with H_new in the loss, with the closure called but
    H_new given no gradient, and with the closure never called."""
    import mhc

    g = torch.Generator(device=DEV).manual_seed(2)
    B, S = 2, 48
    hc = mhc.HyperConnection(D, dynamic=kind != "static", use_fused_weights=kind == "dynamic").to(DEV)
    with torch.no_grad():
        for p in hc.parameters():
            p.add_(_rand(g, *p.shape, scale=0.05))
    H = _rand(g, B, S, 4, D, dtype=dtype)
    bo = _rand(g, B, S, D, dtype=dtype)
    dHn, dbi = _rand(g, B, S, 4, D, dtype=dtype), _rand(g, B, S, D, dtype=dtype)

    def run():
        hc.zero_grad(set_to_none=True)
        Hl, bol = H.clone().requires_grad_(True), bo.clone().requires_grad_(True)
        bi, add = hc(Hl)
        outs, grads, res = [bi], [dbi], {"bi": bi}
        if closure != "never_called":
            Hn = add(bol)
            res["Hn"] = Hn
            if closure == "used":
                outs.append(Hn)
                grads.append(dHn)
        torch.autograd.backward(outs, grads)
        res.update(dH=Hl.grad, dbo=bol.grad)
        res.update({n: p.grad for n, p in hc.named_parameters()})
        return res

    _twice(run)


@pytest.mark.parametrize("B,S,D", [(600, 1, 128), (530, 3, 1024), (512, 5, 4096)])
def test_many_sequences_layer_overwrites_what_it_reads(B, S, D):
    """The dynamic layer's bulk-batch paths: the mean-pool without the projection, the pooled
    rows (at S = 1 H's own rows, with no x kept) projected and differentiated on the MFMA
    kernels in row chunks, and at B = 512, S = 5, D = 4096 pass C at 8 tokens per lane."""
    import mhc

    g = torch.Generator(device=DEV).manual_seed(3)
    hc = mhc.HyperConnection(D).to(DEV)
    with torch.no_grad():
        for p in hc.parameters():
            p.add_(_rand(g, *p.shape, scale=0.05))
    H = _rand(g, B, S, 4, D, dtype=torch.bfloat16)
    bo = _rand(g, B, S, D, dtype=torch.bfloat16)
    dHn, dbi = _rand(g, B, S, 4, D, dtype=torch.bfloat16), _rand(g, B, S, D, dtype=torch.bfloat16)

    def run():
        hc.zero_grad(set_to_none=True)
        Hl, bol = H.clone().requires_grad_(True), bo.clone().requires_grad_(True)
        bi, add = hc(Hl)
        Hn = add(bol)
        torch.autograd.backward([Hn, bi], [dHn, dbi])
        res = {"bi": bi, "Hn": Hn, "dH": Hl.grad, "dbo": bol.grad}
        res.update({n: p.grad for n, p in hc.named_parameters()})
        return res

    _twice(run)
