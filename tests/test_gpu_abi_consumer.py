"""The C ABI from a C++ program with no torch in its process (tests/abi_consumer/layer_step.cpp):
one dynamic HyperConnection layer step through libmhc_hip.so, checked against the float64
oracle layer, and the allocation-free forward checked bit for bit against the workspace one.

The program is built by ``__graft_entry__.build()`` (``make -C tests/abi_consumer``) and runs as
a child process; inputs and outputs pass through files.  Inputs follow the draw order of
test_gpu_module.py from a CPU generator: H, phi, branch_output, dH_new, d_branch_input."""

import os
import struct
import subprocess

import numpy as np
import pytest
import torch

from helpers import rel_err
from oracle import mhc_oracle as O

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
BINARY = os.path.join(HERE, "abi_consumer", "layer_step")
CODES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def _raw(t: torch.Tensor) -> bytes:
    """The tensor's bytes as stored (bf16 / fp16 as 16-bit words)."""
    t = t.contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().tobytes()
    return t.numpy().astype(np.float32).tobytes()


def _from_raw(buf: bytes, off: int, n: int, dtype: torch.dtype):
    e = 4 if dtype == torch.float32 else 2
    chunk = buf[off:off + n * e]
    if dtype == torch.float32:
        arr = np.frombuffer(chunk, dtype=np.float32).astype(np.float64)
    else:
        arr = torch.frombuffer(bytearray(chunk), dtype=torch.int16).view(dtype).to(torch.float64).numpy()
    return arr, off + n * e


@pytest.mark.parametrize("dtype,B,S,D,tol,h_tol", [(torch.bfloat16, 2, 96, 448, 2e-2, 2e-2),
                                                    (torch.float32, 2, 64, 256, 1e-5, 1e-4)])
def test_layer_step_from_cpp(tmp_path, dtype, B, S, D, tol, h_tol):
    if not os.path.exists(BINARY):
        raise AssertionError(f"{BINARY} is not built (make -C tests/abi_consumer, or __graft_entry__.build())")
    g = torch.Generator()
    g.manual_seed(0)
    H = torch.randn((B, S, 4, D), generator=g).to(dtype)
    phi = (torch.randn((24, 4 * D), generator=g) * 0.02).T.contiguous()
    pre_base = torch.tensor([1.0, 0.0, 0.0, 0.0])  # the module's init at layer_idx 0
    post_base = torch.ones(4)
    res_base = torch.eye(4)
    alphas = torch.tensor([0.1, 0.1, 0.1])
    bo = torch.randn((B, S, D), generator=g).to(dtype)
    dHn = torch.randn((B, S, 4, D), generator=g).to(dtype)
    dbi = torch.randn((B, S, D), generator=g).to(dtype)
    iters, eps = 20, 1e-6

    inp = tmp_path / "in.bin"
    out = tmp_path / "out.bin"
    with open(inp, "wb") as f:
        f.write(struct.pack("<5q", CODES[dtype], B, S, D, iters))
        f.write(struct.pack("<d", eps))
        for t in (H, phi, pre_base, post_base, res_base, alphas[0:1], alphas[1:2], alphas[2:3], bo, dHn, dbi):
            f.write(_raw(t))
    print(f"layer_step dtype={dtype} B={B} S={S} D={D}", flush=True)
    run = subprocess.run([BINARY, str(inp), str(out)], capture_output=True, text=True, timeout=120)
    print(run.stdout, run.stderr, flush=True)
    assert run.returncode == 0, run.stderr

    buf = out.read_bytes()
    off = 0
    bi, off = _from_raw(buf, off, B * S * D, dtype)
    Hn, off = _from_raw(buf, off, B * S * 4 * D, dtype)
    dbo, off = _from_raw(buf, off, B * S * D, dtype)
    dH, off = _from_raw(buf, off, B * S * 4 * D, dtype)
    dpost, off = _from_raw(buf, off, B * 4, torch.float32)
    gphi, off = _from_raw(buf, off, 4 * D * 24, torch.float32)
    gbias, off = _from_raw(buf, off, 24, torch.float32)
    galpha, off = _from_raw(buf, off, 3, torch.float32)
    off += (B * 24 + B * 4 * D) * 4  # w and x (their bits are compared inside the program)
    (same,) = struct.unpack("<q", buf[off:off + 8])
    assert off + 8 == len(buf)
    assert same == 1, "the allocation-free forward differs from the workspace forward"

    f64 = lambda t: t.to(torch.float64).numpy()  # noqa: E731
    p = {"phi": f64(phi), "H_pre_base": f64(pre_base), "H_post_base": f64(post_base), "H_res_base": f64(res_base),
         "alpha_pre": f64(alphas[0:1]), "alpha_post": f64(alphas[1:2]), "alpha_res": f64(alphas[2:3])}
    obi, oHn, cache = O.layer_forward(p, f64(H), f64(bo), True, True, iters, eps)
    og = O.layer_backward(p, cache, f64(dHn), f64(dbi))
    errs = {"bi": rel_err(bi.reshape(obi.shape), obi), "H_new": rel_err(Hn.reshape(oHn.shape), oHn),
            "dH": rel_err(dH.reshape(og["H"].shape), og["H"]), "dbo": rel_err(dbo.reshape(og["bo"].shape), og["bo"]),
            "dphi": rel_err(gphi.reshape(og["phi"].shape), og["phi"]),
            "dbias": rel_err(gbias, np.concatenate([np.ravel(og["H_pre_base"]), np.ravel(og["H_post_base"]),
                                                    np.ravel(og["H_res_base"])])),
            "dalpha": rel_err(galpha, np.concatenate([np.ravel(og["alpha_pre"]), np.ravel(og["alpha_post"]),
                                                      np.ravel(og["alpha_res"])]))}
    print("layer_step errors:", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    assert errs["bi"] < tol and errs["H_new"] < tol, errs
    assert errs["dH"] < h_tol and errs["dbo"] < h_tol, errs
    for k in ("dphi", "dbias", "dalpha"):
        assert errs[k] < 1e-4, (k, errs)
    assert np.all(np.isfinite(dpost))
