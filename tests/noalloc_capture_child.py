"""Child process of tests/test_zz_no_alloc.py::test_noalloc_first_call_under_graph_capture.

In a fresh process, the first call of mhc_layer_dynamic_forward_noalloc (and the first launch
of any kernel of the library) happens inside torch.cuda.graph capture.  The graph is replayed
three times, the outputs filled with NaN before each replay, and each replay must give the
bits of mhc_layer_dynamic_forward (with a workspace, called eagerly afterwards).  Exit status
0 on success; the reason is printed otherwise.
"""

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path[:0] = [os.path.join(ROOT, "mhc-triton_amd"), ROOT]

import torch  # noqa: E402

from mhc import _lib  # noqa: E402

DEV = "cuda"


def main() -> int:
    B, S, D, dtype = 3, 96, 512, torch.bfloat16
    g = torch.Generator(device=DEV).manual_seed(21)
    H = torch.randn((B, S, 4, D), generator=g, device=DEV).to(dtype)
    phi = torch.randn((4 * D, 24), generator=g, device=DEV) * 0.02
    base = [torch.randn(4, generator=g, device=DEV), torch.randn(4, generator=g, device=DEV),
            torch.randn((4, 4), generator=g, device=DEV)]
    alphas = [torch.rand(1, generator=g, device=DEV) * 0.5 for _ in range(3)]

    def outputs():
        return (torch.empty((B, S, D), device=DEV, dtype=dtype), torch.empty((B, 4 * D), device=DEV),
                torch.empty((B, 24), device=DEV), torch.empty((B, 25), device=DEV))

    def args(outs):
        return [H.data_ptr(), _lib.dtype_code(H), phi.data_ptr(), *[t.data_ptr() for t in base],
                *[a.data_ptr() for a in alphas], *[o.data_ptr() for o in outs], B, S, D, 20, 1e-6]

    lib = _lib.load()
    got = outputs()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib.mhc_layer_dynamic_forward_noalloc(*args(got), torch.cuda.current_stream().cuda_stream)
    if rc != 0:
        print(f"noalloc call under capture returned {rc}: {lib.mhc_last_error().decode()}", flush=True)
        return 1
    ref = outputs()
    ws = torch.empty(lib.mhc_layer_workspace_bytes(B, S, D, _lib.dtype_code(H)), dtype=torch.uint8, device=DEV)
    rc = lib.mhc_layer_dynamic_forward(*args(ref), ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
    if rc != 0:
        print(f"workspace call returned {rc}: {lib.mhc_last_error().decode()}", flush=True)
        return 1
    for replay in range(3):
        for t in got:
            t.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("branch_input", "x", "w", "aux"), ref, got):
            if not torch.equal(a, b):
                print(f"replay {replay}: {name} differs from the workspace forward", flush=True)
                return 1
        print(f"replay {replay}: bit-identical", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
