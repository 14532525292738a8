"""The streaming-ceiling probe (libmhc_probe.so, `bench.py --stream-ceiling`) moves the bytes
it is credited with: every input row of a mix is read and every output row written, with the
values its kernel defines (output row o = the 32-bit sum of all input rows, plus o in the first
word, plus input row o mod n), on whole 4 KiB tiles and on flattened items.  A probe that
dropped a load would report a ceiling for a lighter mix than the layer kernel it is compared
with.
"""

import ctypes
import os

import pytest
import torch

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROBE = os.path.join(ROOT, "mhc-triton_amd", "probe", "libmhc_probe.so")
MIXES = [(1, 0, 0, 0), (0, 0, 0, 1), (1, 0, 0, 1), (4, 0, 0, 0), (4, 0, 0, 1), (4, 1, 0, 4), (4, 1, 0, 1),
         (4, 4, 1, 0), (4, 0, 0, 5), (1, 0, 0, 4), (4, 4, 1, 4)]


@pytest.fixture(scope="module")
def probe():
    if not os.path.exists(PROBE):
        pytest.fail(f"{PROBE} is not built (make -C mhc-triton_amd)")
    lib = ctypes.CDLL(PROBE)
    fn = lib.mhc_probe_stream
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int] * 4 + [ctypes.c_void_p] * 4 + [ctypes.c_int64] * 2 + [ctypes.c_int] * 2 + \
        [ctypes.c_void_p] * 2
    return fn


@pytest.mark.parametrize("mix", MIXES, ids=lambda m: "".join(map(str, m)))
@pytest.mark.parametrize("nt,cap,row_bytes", [(1, 2, 8192), (0, 0, 8192), (1, 3, 14336), (1, 0, 1040)],
                         ids=["tiles-nt", "tiles-plain", "flat-14336", "flat-1040"])
def test_probe_moves_every_row(probe, mix, nt, cap, row_bytes):
    na, nb, nc, nw = mix
    tokens = 37
    words = row_bytes // 4
    g = torch.Generator(device="cuda")
    g.manual_seed(sum(mix) * 7 + nt)

    def arr(rows):
        return torch.randint(0, 2 ** 31 - 1, (tokens, max(rows, 1), words), generator=g, device="cuda",
                             dtype=torch.int32)

    a, b, c = arr(na), arr(nb), arr(nc)
    w = torch.full((tokens, max(nw, 1), words), -7, dtype=torch.int32, device="cuda")
    sink = torch.zeros(256, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    rc = probe(na, nb, nc, nw, a.data_ptr(), b.data_ptr(), c.data_ptr(), w.data_ptr(), tokens, row_bytes, cap, nt,
               sink.data_ptr(), stream)
    assert rc == 0
    torch.cuda.synchronize()
    rows = [a[:, i] for i in range(na)] + [b[:, i] for i in range(nb)] + [c[:, i] for i in range(nc)]
    mask = (1 << 32) - 1
    tot = torch.zeros((tokens, words), dtype=torch.int64, device="cuda")
    for r in rows:
        tot = (tot + (r.to(torch.int64) & mask)) & mask
    for o in range(nw):
        ref = tot.clone()
        ref[:, 0::4] = (ref[:, 0::4] + o) & mask  # the first word of each 16-byte vector
        if rows:
            ref = (ref + (rows[o % len(rows)].to(torch.int64) & mask)) & mask
        got = w[:, o].to(torch.int64) & mask
        assert torch.equal(got, ref), f"output row {o}"
    if nw == 0:
        assert int(sink.abs().sum()) == 0  # the store that keeps the loads live never fires here


@pytest.mark.parametrize("mode", [1, 2, 3])
@pytest.mark.parametrize("R,K,rows", [(1000, 512, 300), (256, 768, 64)])
def test_dynw_backward_probe_copies_every_strip(mode, R, K, rows):
    """bench.py --dynw-ceiling's backward pattern (the MFMA backward's 512-byte strips, 64-row
    blocks, two blocks in flight) reads every element of x and writes every element of grad_x:
    copied with the first word of each 16-byte vector XOR 1 (mode 1), or unchanged through the
    LDS tiles (modes 2 and 3).  Row chunks end inside a block."""
    lib = ctypes.CDLL(PROBE)
    fn = lib.mhc_probe_dynw
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int, ctypes.c_int] + [ctypes.c_void_p] * 2 + [ctypes.c_int64] * 3 + [ctypes.c_void_p] * 2
    g = torch.Generator(device="cuda").manual_seed(R + mode)
    x = torch.randint(-2 ** 15, 2 ** 15 - 1, (R, K), generator=g, device="cuda", dtype=torch.int16)
    gx = torch.full_like(x, -7)
    sink = torch.zeros(256, dtype=torch.int32, device="cuda")
    assert fn(1, mode, x.data_ptr(), gx.data_ptr(), R, K, rows, sink.data_ptr(),
              torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    want = x.view(torch.int32).reshape(R, K // 8, 4).clone()
    if mode == 1:
        want[:, :, 0] ^= 1
    assert torch.equal(gx.view(torch.int32).reshape(R, K // 8, 4), want)


@pytest.mark.parametrize("mode", [3, 4])
@pytest.mark.parametrize("R,K,rows", [(1000, 2048, 320), (96, 1040, 64)])
def test_dynw_forward_probe_writes_every_record(mode, R, K, rows):
    """The forward pattern's modes 3 and 4 write one 25-float record per row and K chunk, as the
    projection kernel does: its tile loop covers every row of every range."""
    lib = ctypes.CDLL(PROBE)
    fn = lib.mhc_probe_dynw
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int, ctypes.c_int] + [ctypes.c_void_p] * 2 + [ctypes.c_int64] * 3 + [ctypes.c_void_p] * 2
    nK = (K // 16 + 63) // 64
    x = torch.ones((R, K), device="cuda", dtype=torch.bfloat16)
    part = torch.full((R * nK * 25,), float("nan"), device="cuda")
    sink = torch.zeros(256, dtype=torch.int32, device="cuda")
    assert fn(0, mode, x.data_ptr(), part.data_ptr(), R, K, rows, sink.data_ptr(),
              torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    assert not part.isnan().any()
