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
PROBE = os.path.join(ROOT, "mhc-triton_amd", "mhc", "libmhc_probe.so")
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
