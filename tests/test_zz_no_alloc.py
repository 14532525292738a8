"""mhc_layer_dynamic_forward_noalloc (no reference counterpart: the dynamic layer forward for
callers that cannot allocate device memory) against mhc_layer_dynamic_forward, through the
C ABI: the same bits for branch_input, x, w and aux, on two calls in a row (the second with a
smaller input, so the static scratch still holds the first call's partials), and the
documented rejection of a shape whose scratch exceeds the static array."""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _inputs(B, S, D, dtype, seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    H = torch.randn((B, S, 4, D), generator=g, device=DEV).to(dtype)
    phi = torch.randn((4 * D, 24), generator=g, device=DEV) * 0.02
    base = [torch.randn(4, generator=g, device=DEV), torch.randn(4, generator=g, device=DEV),
            torch.randn((4, 4), generator=g, device=DEV)]
    alphas = [torch.rand(1, generator=g, device=DEV) * 0.5 for _ in range(3)]
    return H, phi, base, alphas


def _outputs(B, S, D, dtype):
    return (torch.empty((B, S, D), device=DEV, dtype=dtype), torch.empty((B, 4 * D), device=DEV),
            torch.empty((B, 24), device=DEV), torch.empty((B, 25), device=DEV))


def _call(lib, noalloc, H, phi, base, alphas, outs, iters=20, eps=1e-6):
    from mhc import _lib

    B, S, _, D = H.shape
    args = [H.data_ptr(), _lib.dtype_code(H), phi.data_ptr(), *[t.data_ptr() for t in base],
            *[a.data_ptr() for a in alphas], *[o.data_ptr() for o in outs], B, S, D, iters, eps]
    st = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = lib.mhc_layer_dynamic_forward_noalloc(*args, st)
    else:
        ws = torch.empty(lib.mhc_layer_workspace_bytes(B, S, D, _lib.dtype_code(H)), dtype=torch.uint8, device=DEV)
        rc = lib.mhc_layer_dynamic_forward(*args, ws.data_ptr(), ws.numel(), st)
        torch.cuda.synchronize()
    return rc


@pytest.mark.parametrize("first,second", [
    ((4, 512, 1024, torch.bfloat16), (2, 100, 256, torch.bfloat16)),
    ((3, 257, 640, torch.float16), (1, 33, 100, torch.float32)),
])
def test_noalloc_forward_matches_workspace_forward(first, second):
    from mhc import _lib

    lib = _lib.load()
    for i, (B, S, D, dtype) in enumerate((first, second)):
        print(f"noalloc call {i}: B={B} S={S} D={D} {dtype}", flush=True)
        H, phi, base, alphas = _inputs(B, S, D, dtype, seed=10 + i)
        ref, got = _outputs(B, S, D, dtype), _outputs(B, S, D, dtype)
        assert _call(lib, False, H, phi, base, alphas, ref) == 0, lib.mhc_last_error()
        assert _call(lib, True, H, phi, base, alphas, got) == 0, lib.mhc_last_error()
        torch.cuda.synchronize()
        for name, a, b in zip(("branch_input", "x", "w", "aux"), ref, got):
            assert torch.equal(a, b), (i, name)


def test_noalloc_rejects_shapes_beyond_the_scratch():
    """B = 512 at D = 4096 needs about 37 MB of column partials: the call returns
    MHC_ERR_WORKSPACE (3) with a message, before any device work; the workspace entry
    point runs the same shape."""
    from mhc import _lib

    lib = _lib.load()
    B, S, D = 512, 1, 4096
    H, phi, base, alphas = _inputs(B, S, D, torch.bfloat16, seed=3)
    outs = _outputs(B, S, D, torch.bfloat16)
    assert _call(lib, True, H, phi, base, alphas, outs) == 3
    assert b"static array holds" in lib.mhc_last_error()
    assert _call(lib, False, H, phi, base, alphas, outs) == 0


def test_noalloc_first_call_under_graph_capture():
    """The first noalloc call of a process (which looks up the scratch array's device address)
    made inside torch.cuda.graph capture: in a child process, so that no earlier call has
    resolved the address or loaded the library's kernels.  Replays match the workspace entry
    point bit for bit (tests/noalloc_capture_child.py)."""
    import os
    import subprocess
    import sys

    child = os.path.join(os.path.dirname(os.path.abspath(__file__)), "noalloc_capture_child.py")
    run = subprocess.run([sys.executable, child], capture_output=True, text=True, timeout=180)
    print(run.stdout, run.stderr[-2000:], flush=True)
    assert run.returncode == 0, run.stdout + run.stderr[-2000:]
