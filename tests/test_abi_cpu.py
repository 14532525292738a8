"""The C-ABI boundary, checked without a GPU: the library loads, exports every
function include/mhc_abi.h declares, the ctypes binding agrees with the header
on arity, and host-side argument validation returns the documented status
codes before any device work.
"""

import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mhc_abi.h")


def _declared():
    """{name: n_args} for every function prototype in the header."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(?:int|size_t|const char\*)\s+(mhc_\w+)\s*\(([^)]*)\)\s*;", text):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else len(args.split(","))
    return out


@pytest.fixture(scope="module")
def lib():
    from mhc import _lib

    if not os.path.exists(_lib.LIB_PATH):
        import __graft_entry__

        __graft_entry__.build()
    return _lib.load()


def test_header_declares_the_expected_surface():
    names = set(_declared())
    for op in ("sinkhorn_forward", "sinkhorn_backward", "stream_mix_forward", "stream_mix_backward",
               "add_residual_forward", "add_residual_backward", "dynamic_weights_forward",
               "dynamic_weights_backward", "layer_dynamic_forward", "layer_dynamic_backward"):
        assert "mhc_" + op in names


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), name


def test_ctypes_binding_matches_header_arity():
    from mhc import _lib

    decl = _declared()
    assert set(decl) == set(_lib._SIGNATURES)
    for name, n in decl.items():
        assert len(_lib._SIGNATURES[name][1]) == n, name


def test_version_and_workspace_queries(lib):
    from mhc import _lib

    assert lib.mhc_abi_version() == _lib.ABI_VERSION
    assert lib.mhc_stream_mix_backward_workspace_bytes(4, 4096, 4096, 1) > 0
    assert lib.mhc_add_residual_backward_workspace_bytes(4, 4096, 4096, 1) > 0
    assert lib.mhc_dynamic_weights_workspace_bytes(0, 16384) == 0
    ws = lib.mhc_layer_workspace_bytes(4, 4096, 4096, 1)
    # grad_x [B, 4D] f32 dominates: at least 256 KiB here, and 256-byte granular
    assert ws >= 4 * 4 * 4096 * 4 and ws % 256 == 0
    # The backward passes that run one workgroup per tile keep one partial record
    # per tile: 256 lanes x one 16-byte vector, sized for the narrowest (fp32, 4
    # elements); 20 floats for the mixing backward, 4 for the closure backward.
    for B, S, D in ((4, 4096, 4096), (1, 8192, 7168), (16, 2048, 2048), (3, 5, 12)):
        tiles = (S * D // 4 + 255) // 256
        assert lib.mhc_stream_mix_backward_workspace_bytes(B, S, D, 1) >= B * tiles * 20 * 4
        assert lib.mhc_add_residual_backward_workspace_bytes(B, S, D, 1) >= B * tiles * 4 * 4
        assert lib.mhc_layer_workspace_bytes(B, S, D, 1) >= B * tiles * 20 * 4 + B * 4 * D * 4


def test_host_side_validation_without_gpu(lib):
    # negative sizes, bad dtype codes, missing workspace: rejected before any launch
    assert lib.mhc_sinkhorn_forward(None, None, -1, 0, 20, 1e-8, None) == 1
    assert lib.mhc_sinkhorn_forward(None, None, 0, 0, 20, 1e-8, None) == 0  # empty is a no-op
    assert lib.mhc_sinkhorn_forward(None, None, 4, 0, -3, 1e-8, None) == 1
    assert lib.mhc_stream_mix_forward(None, None, None, None, None, 2, 3, 4, 0, None) == 1  # null pointers
    assert lib.mhc_stream_mix_forward(None, None, None, None, None, 0, 3, 4, 0, None) == 0
    assert lib.mhc_stream_mix_forward(16, 16, 16, 16, 16, 2, 3, 4, 7, None) == 2  # dtype 7
    assert b"dtype" in lib.mhc_last_error()
    assert lib.mhc_stream_mix_backward(16, 16, 16, 16, 16, 16, 16, 16, 2, 3, 4, 0, None, 0, None) == 3
    assert b"workspace" in lib.mhc_last_error()
    assert lib.mhc_stream_mix_forward(16, 16, 16, 16, 16, 1, 1 << 20, 1 << 13, 0, None) == 1  # S*D >= 2^32
    # just under 2^32: the last tile's first index would wrap a 32-bit counter
    assert lib.mhc_stream_mix_forward(16, 16, 16, 16, 16, 1, (1 << 32) - 1, 1, 0, None) == 1
    assert b"2^32 - 2^16" in lib.mhc_last_error()
    assert lib.mhc_layer_dynamic_forward(None, 0, *([None] * 11), 1, 1, 1, -1, 1e-6, None, 0, None) == 1
    # the allocation-free forward: a shape whose scratch exceeds the static array is refused
    # with MHC_ERR_WORKSPACE before any HIP call (B = 512 at D = 4096 needs ~37 MB)
    assert lib.mhc_layer_dynamic_forward_noalloc(16, 1, *([16] * 11), 512, 1, 4096, 20, 1e-6, None) == 3
    assert b"static array holds" in lib.mhc_last_error()
    assert lib.mhc_layer_dynamic_forward_noalloc(None, 1, *([None] * 11), 2, 3, 4, 20, 1e-6, None) == 1


def test_ops_reject_cpu_tensors():
    import mhc

    M = torch.randn(2, 4, 4)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        mhc.sinkhorn_knopp(M)
    H = torch.randn(1, 2, 4, 8)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        mhc.fused_stream_mix(H, torch.rand(1, 4), torch.rand(1, 4, 4))
    hc = mhc.HyperConnection(8)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        hc(H)


def test_shape_errors_are_assertion_compatible():
    import mhc

    with pytest.raises(AssertionError):
        mhc.sinkhorn_knopp(torch.zeros(2, 4, 5))
    with pytest.raises(AssertionError):
        mhc.fused_dynamic_weights(torch.zeros(2, 8), torch.zeros(8, 23), torch.zeros(24),
                                  torch.ones(1), torch.ones(1), torch.ones(1))
    with pytest.raises(ValueError):
        mhc.HyperConnection(8, num_streams=3)
    with pytest.raises(ValueError):
        mhc.HyperConnection(8)(torch.zeros(1, 2, 4, 9))


def test_stream_ceiling_probe_rejects_bad_shapes_without_gpu(lib):
    """libmhc_probe.so (bench.py --stream-ceiling) is separate from the mHC C ABI: it exports only
    its probe, and refuses unsupported mixes and shapes before any device work."""
    import ctypes

    path = os.path.join(ROOT, "mhc-triton_amd", "probe", "libmhc_probe.so")
    if not os.path.exists(path):
        import __graft_entry__

        __graft_entry__.build()
    probe = ctypes.CDLL(path)
    fn = probe.mhc_probe_stream
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int] * 4 + [ctypes.c_void_p] * 4 + [ctypes.c_int64] * 2 + [ctypes.c_int] * 2 + \
        [ctypes.c_void_p] * 2
    null = None
    fake = 4096  # never dereferenced: every call below is refused on the host
    assert fn(1, 0, 0, 1, fake, null, null, fake, 0, 8192, 0, 1, null, null) == 1  # no tokens
    assert fn(1, 0, 0, 1, fake, null, null, fake, 16, 1000, 0, 1, null, null) == 1  # row not a multiple of 16 bytes
    assert fn(1, 0, 0, 1, null, null, null, fake, 16, 8192, 0, 1, null, null) == 1  # missing input array
    assert fn(1, 0, 0, 0, fake, null, null, null, 16, 8192, 0, 1, null, null) == 1  # read-only mix without a sink
    assert fn(2, 0, 0, 0, fake, null, null, null, 16, 8192, 0, 1, fake, null) == 1  # unsupported mix
    assert fn(4, 0, 0, 0, fake, null, null, null, 16, 1 << 30, 0, 1, fake, null) == 1  # span >= 2^31
    assert not hasattr(lib, "mhc_probe_stream")
