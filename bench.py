#!/usr/bin/env python3
"""mHC layer forward+backward throughput on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload config3]
    python bench.py --ops        # the low-level ops one by one (one JSON line)
    python bench.py --readme     # the reference's own benchmark table, same workloads
    python bench.py --dynw-ceiling   # access-pattern ceilings of the MFMA dynamic-weights kernels
    python bench.py --decode     # short sequences, from 1 to 4096 of them: HIP-graph step latency

One "step" is the HyperConnection layer's forward and backward over one
synthetic batch, exactly as a transformer block uses it:

    bi, add = hc(H); H_new = add(bo)
    torch.autograd.backward([H_new, bi], [dH_new, d_bi])

with ``H`` and ``bo`` leaves (so dH and d_bo are produced) and every parameter
gradient computed.  Gradients are reset to None before each step, as an
optimizer's ``zero_grad(set_to_none=True)`` would, so no step pays for gradient
accumulation.  Inputs are resident in HBM before the timed region.

Printed: one JSON line (metric, value = tokens/s of the whole job, roofline of
the dominant kernel measured with HIP events on the stream it runs on, the CPU
baseline of the reference's PyTorch path timed on this host).  The default
config3 run also times configs 4 and 5 (GPU legs only) and reports them under
"workloads", with config 2 (Sinkhorn) and the dynamic-weights op at R = tokens
under "workloads.ops"; --no-workloads skips them.

Workloads (reference benchmark shapes, src/mhc/module.py layer):
  config3  dim 4096 bf16, B=4 S=4096, dynamic fused weights (the headline)
  config4  dim 7168 bf16, B=1 S=8192, dynamic fused weights
  config5  dim 2048 fp16, B=16 S=2048, static weights
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "mhc-triton_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "mHC layer fwd+bwd tokens/sec at dim 4096 bf16; achieved HBM GB/s vs roofline"
HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, GB/s

WORKLOADS = {
    "config3": dict(B=4, S=4096, D=4096, dtype="bf16", dynamic=True),
    "config4": dict(B=1, S=8192, D=7168, dtype="bf16", dynamic=True),
    "config5": dict(B=16, S=2048, D=2048, dtype="fp16", dynamic=False),
}

# Algorithmic HBM bytes per token, in units of D * e (e = element size of H):
# the dependency-forced minimum of the layer behind this API.
#   dynamic forward 18: mean-pool reads H (4); branch_input reads H (4), writes
#       bi (1); H_new reads H (4) and bo (1), writes H_new (4)
#   dynamic backward 24: closure backward reads dH_new (4) and bo (1), writes
#       d_bo (1); weight-gradient pass reads d_bi (1), dH_new (4), H (4);
#       dH pass reads d_bi (1), dH_new (4), writes dH (4)
#   static: no mean-pool (14 forward) and one backward pass for the weight
#       gradients and dH (19).
ALGO_UNITS = {True: (18, 24), False: (14, 19)}

# HBM bytes one launch of the closure-forward kernel moves, measured with two
# rocprofv3 counter passes over this bench (`--pmc FETCH_SIZE`, then
# `--pmc WRITE_SIZE`), each scaled by what the counter reads for a 512 MiB
# device copy (`bench.py --calibrate-copy`: FETCH_SIZE x2.0, WRITE_SIZE x1.0 on
# MI355X).  Measured at commit TRAFFIC_COMMIT on the kernel as built there;
# algorithmic bytes 9 D e T: config3 1,207,959,552 (+0.018%), config4
# 1,056,964,608 (+0.018%), config5 1,207,959,552 (+0.012%).
MEASURED_TRAFFIC = {"config3": 1208180457, "config4": 1057155147, "config5": 1208107132}
TRAFFIC_COMMIT = "bd0c8b8"

# Best fraction of 8 TB/s that a kernel of the closure forward's launch shape
# reaches when it only moves the same 5:4 read / write mix (4 H rows + bo read,
# 4 H_new rows written per token) at the config-3 layout: `bench.py
# --stream-ceiling` (profiles/stream_ceiling.md).  Row layouts that are not a
# whole number of 4 KiB tiles (config 4) are not measured.
STREAM_CEILING_5_4 = {"config3": 0.814, "config5": None, "config4": None}


def _log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="config3", choices=sorted(WORKLOADS))
    ap.add_argument("--no-workloads", action="store_true",
                    help="skip the GPU legs that the default (config3) run adds under 'workloads': configs "
                         "4 and 5, and 'ops' (config-2 Sinkhorn, dynamic weights at R = K = 16384 bf16)")
    ap.add_argument("--cpu-reps", type=int, default=3,
                    help="timed runs of the cpu_baseline leg at the workload's shape, after one warm-up "
                         "(0 disables it)")
    ap.add_argument("--ops", action="store_true",
                    help="time the low-level ops one by one (config-2 Sinkhorn, the stream ops and "
                         "expand / collapse at config-3 size, dynamic weights) and exit")
    ap.add_argument("--readme", action="store_true",
                    help="run the reference's published benchmark table (README.md:183-202, made by "
                         "benchmarks/benchmark.py) on this build: same workloads, same timing method, "
                         "beside the published H100 numbers, and exit")
    ap.add_argument("--dynw-ceiling", action="store_true",
                    help="time probe kernels with the access patterns of the MFMA dynamic-weights kernels "
                         "(forward and backward, R = K = 16384 bf16), adding the kernels' costs one at a time, "
                         "and the op itself in the same run")
    ap.add_argument("--decode", action="store_true",
                    help="time the dynamic layer at short sequences (S = 1 and 8, B from 1 to 4096, dim 4096 "
                         "bf16) as replayed HIP graphs: the no-grad forward with the closure, and forward + "
                         "backward, and exit")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run 3 plain device copies of 512 MiB (the known-size kernel that scales "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE readings into bytes) and exit")
    ap.add_argument("--stream-ceiling", action="store_true",
                    help="only time the streaming-ceiling probe (libmhc_probe.so): kernels shaped like the "
                         "layer's streaming kernels that move the same read / write mixes at the workload's "
                         "layout and do nothing else, over occupancy caps and cache policies, and exit")
    return ap.parse_args()


COPY_BYTES = 512 << 20

KERNEL_SAMPLE_EVERY = 5  # timed steps per live event-timed launch of the dominant kernel

# (mix, input rows per token in three arrays, output rows, layer kernels with that mix)
PROBE_MIXES = [
    ("read 1:0", (1, 0, 0), 0, "plain read"),
    ("write 0:1", (0, 0, 0), 1, "plain write"),
    ("copy 1:1", (1, 0, 0), 1, "plain copy"),
    ("4:0", (4, 0, 0), 0, "colsum_kernel (mean-pool)"),
    ("4:1", (4, 0, 0), 1, "mix_fwd_kernel<BI> (branch_input)"),
    ("5:4", (4, 1, 0), 4, "mix_fwd_kernel<RES,ADD_BO> (closure forward); dh_kernel (pass C)"),
    ("5:1", (4, 1, 0), 1, "add_residual_bwd_kernel (closure backward)"),
    ("9:0", (4, 4, 1), 0, "mix_bwd_kernel<REDUCE> (pass B)"),
    ("4:5", (4, 0, 0), 5, "fused_stream_mix forward (H_residual and branch_input)"),
    ("1:4", (1, 0, 0), 4, "expand_streams"),
    ("9:4", (4, 4, 1), 4, "fused_stream_mix backward (dH with the dH_pre / dH_res partials)"),
]


def _stream_ceiling(tokens: int, row_bytes: int, caps=(0, 2, 3, 4, 6, 8), reps: int = 20,
                    warm: int = 3) -> dict:
    """Best HBM rate of each read / write mix of the layer's streaming kernels, as moved by a kernel of the
    same launch shape (one 16-byte vector per lane and row, buffer resources, one tile or 256 flattened
    items per workgroup) that computes nothing: the ceiling those kernels are measured against.  The
    workload's layout: T tokens of D * e byte rows; the one-row mixes run over 4 T tokens."""
    import ctypes

    import torch

    path = os.path.join(ROOT, "mhc-triton_amd", "probe", "libmhc_probe.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built (make -C mhc-triton_amd)")
    lib = ctypes.CDLL(path)
    fn = lib.mhc_probe_stream
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int] * 4 + [ctypes.c_void_p] * 4 + [ctypes.c_int64] * 2 + [ctypes.c_int] * 2 + \
        [ctypes.c_void_p] * 2
    dev = "cuda:0"
    sink = torch.zeros(256, dtype=torch.int32, device=dev)
    out = {}
    for name, (na, nb, nc), nw, kernels in PROBE_MIXES:
        toks = tokens * (4 if na + nb + nc + nw <= 2 else 1)

        def arr(rows):
            return torch.zeros(max(rows, 1) * toks * row_bytes // 4, dtype=torch.int32, device=dev)

        a, b, c, w = arr(na), arr(nb), arr(nc), arr(nw)
        nbytes = toks * (na + nb + nc + nw) * row_bytes
        stream = torch.cuda.current_stream().cuda_stream

        def launch(cap, nt):
            rc = fn(na, nb, nc, nw, a.data_ptr(), b.data_ptr(), c.data_ptr(), w.data_ptr(), toks, row_bytes,
                    cap, nt, sink.data_ptr(), stream)
            if rc:
                raise RuntimeError(f"mhc_probe_stream({name}) returned {rc}")

        runs = {}
        for nt in (1, 0):
            for cap in caps:
                for _ in range(warm):
                    launch(cap, nt)
                ev0 = torch.cuda.Event(enable_timing=True)
                ev1 = torch.cuda.Event(enable_timing=True)
                ev0.record()
                for _ in range(reps):
                    launch(cap, nt)
                ev1.record()
                torch.cuda.synchronize()
                us = ev0.elapsed_time(ev1) * 1e3 / reps
                runs[f"{'nt' if nt else 'plain'} cap{cap}"] = {
                    "us": round(us, 1), "frac": round(nbytes / (us * 1e-6) / (HBM_PEAK_GBS * 1e9), 4)}
        best = max(runs, key=lambda k: runs[k]["frac"])
        out[name] = {"layer_kernels": kernels, "bytes": nbytes, "best": best, **runs[best], "runs": runs}
        _log(f"stream ceiling {name}: best {best} {runs[best]['us']} us {runs[best]['frac']:.3f}")
        del a, b, c, w
        torch.cuda.empty_cache()
    return out


DYNW_FWD_MODES = {0: "loads only", 1: "+ LDS staging and fragment reads", 2: "+ one workgroup barrier per tile",
                  3: "+ split-K records (32 rows x 25 floats per tile and K chunk)",
                  4: "+ the same records chunk-major, stored as 16-byte vectors"}
DYNW_BWD_MODES = {0: "read only", 1: "copy (each vector stored back in place to grad_x)",
                  2: "copy through LDS tiles with two barriers per block",
                  3: "copy through LDS tiles doubled by block parity, both blocks of a pair stored together"}


def _dynw_ceiling(R: int = 16384, K: int = 16384, reps: int = 10, warm: int = 2, rounds: int = 3) -> dict:
    """Probe kernels (csrc/probe/dynw_ceiling.hip) with the grids, per-lane loads, register pipelines
    and LDS reservations of dynw_mfma_kernel and dynw_bwd_mfma_kernel at the op's plan for R = K,
    each mode adding one of the kernels' costs, and the op's forward and backward launchers beside
    them.  The box's kernel times drift by 10-20% over seconds of back-to-back streaming, so the
    probes and the launchers alternate in rounds and each figure is the median over rounds; a
    rocprofv3 kernel trace of this run splits the launchers' time into their kernels."""
    import ctypes

    import torch

    from mhc import _backward as KB
    from mhc import _kernels as KF

    path = os.path.join(ROOT, "mhc-triton_amd", "probe", "libmhc_probe.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built (make -C mhc-triton_amd)")
    lib = ctypes.CDLL(path)
    fn = lib.mhc_probe_dynw
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int, ctypes.c_int] + [ctypes.c_void_p] * 2 + [ctypes.c_int64] * 3 + \
        [ctypes.c_void_p] * 2
    dev = "cuda:0"
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn((R, K), generator=g, device=dev).to(torch.bfloat16)
    gx = torch.empty_like(x)
    nK = (K // 16 + 63) // 64
    part = torch.empty(R * nK * 25, device=dev)
    sink = torch.zeros(256, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    xbytes = R * K * 2
    # the ops' plans at R = K = 16384 (csrc/dynamic_weights.hip): 16 row ranges of 1024 rows per K
    # chunk forward, 4 row chunks of 4096 rows per 256-column block backward
    tiles = (R + 31) // 32
    ngr = min(tiles, (256 + nK - 1) // nK)
    fwd_rows = 32 * ((tiles + ngr - 1) // ngr)
    bwd_rows = (R + 3) // 4

    def timed(call):
        for _ in range(warm):
            call()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1 << 20)  # the host queues the first calls while this spins
        e0.record()
        for _ in range(reps):
            call()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps

    def probe(pattern, mode, out, rows):
        def call():
            rc = fn(pattern, mode, x.data_ptr(), out.data_ptr() if out is not None else None, R, K, rows,
                    sink.data_ptr(), stream)
            if rc:
                raise RuntimeError(f"mhc_probe_dynw({pattern}, {mode}) returned {rc}")
        return call

    phi = torch.randn((K, 24), generator=g, device=dev) * 0.02
    bias = torch.randn(24, generator=g, device=dev)
    al = [torch.tensor([0.1], device=dev) for _ in range(3)]
    gw = [torch.randn(s, generator=g, device=dev) for s in ((R, 4), (R, 4), (R, 4, 4))]
    H_pre, _, _, aux = KF.fused_dynamic_weights_forward(x, phi, bias, *al, return_aux=True)

    def fwd():
        KF.fused_dynamic_weights_forward(x, phi, bias, *al)

    def bwd():
        KB.fused_dynamic_weights_backward(x, phi, bias, al, aux, H_pre, *gw, 20, 1e-6)

    t = {}
    for rnd in range(rounds):
        for mode in DYNW_FWD_MODES:
            t.setdefault(("forward", mode), []).append(timed(probe(0, mode, part, fwd_rows)))
        t.setdefault(("op", "forward"), []).append(timed(fwd))
        for mode in DYNW_BWD_MODES:
            t.setdefault(("backward", mode), []).append(timed(probe(1, mode, gx, bwd_rows)))
        t.setdefault(("op", "backward"), []).append(timed(bwd))
        _log(f"dynw ceiling round {rnd + 1}/{rounds}: " +
             ", ".join(f"{k[0]} {k[1]} {v[-1]:.1f}" for k, v in t.items()))
    med = {k: statistics.median(v) for k, v in t.items()}
    res = {"forward": {}, "backward": {}}
    for mode, what in DYNW_FWD_MODES.items():
        us = med[("forward", mode)]
        res["forward"][str(mode)] = {"what": what, "us": round(us, 1),
                                     "frac": round(xbytes / (us * 1e-6) / (HBM_PEAK_GBS * 1e9), 4)}
    for mode, what in DYNW_BWD_MODES.items():
        us = med[("backward", mode)]
        nbytes = xbytes * (1 if mode == 0 else 2)
        res["backward"][str(mode)] = {"what": what, "us": round(us, 1),
                                      "frac": round(nbytes / (us * 1e-6) / (HBM_PEAK_GBS * 1e9), 4)}
    res["op"] = {"forward_us": round(med[("op", "forward")], 1), "backward_us": round(med[("op", "backward")], 1),
                 "note": "launcher calls (all of each op's kernels); per-kernel times come from a kernel trace"}
    res["plan"] = {"R": R, "K": K, "forward_rows_per_workgroup": fwd_rows, "k_chunks": nK,
                   "backward_rows_per_chunk": bwd_rows, "x_bytes": xbytes, "rounds": rounds,
                   "launches_per_figure": reps}
    return res


def _calibrate_copy() -> int:
    import torch

    src = torch.ones(COPY_BYTES // 2, dtype=torch.bfloat16, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "device copy", "bytes_read": COPY_BYTES, "bytes_written": COPY_BYTES,
                      "launches": 3}), flush=True)
    return 0


def _decode_leg(D: int = 4096, reps: int = 5, calls: int = 30) -> dict:
    """The dynamic HyperConnection layer at short sequences (decode, batched decode, short-sequence
    training), each step captured in a HIP graph and replayed `calls` times, `reps` times over:
    the median per-replay wall time of the no-grad forward with its closure (what a serving loop
    runs) and of the forward + backward.  Replays are launch-bound at the small shapes, so the
    figure is latency, not bandwidth; `frac` is the algorithmic bytes (18 D e per token forward,
    42 with the backward) over the time, against 8 TB/s."""
    import torch

    import mhc

    out = {}
    for B, S in ((1, 1), (8, 1), (64, 1), (512, 1), (4096, 1), (64, 8), (512, 8)):
        torch.manual_seed(0)
        hc = mhc.HyperConnection(D).to("cuda")
        with torch.no_grad():
            hc.phi.normal_(0.0, 0.02)
        params = list(hc.parameters())
        H = torch.randn(B, S, 4, D, device="cuda").bfloat16().requires_grad_(True)
        bo = torch.randn(B, S, D, device="cuda").bfloat16().requires_grad_(True)
        dHn = torch.randn(B, S, 4, D, device="cuda").bfloat16()
        dbi = torch.randn(B, S, D, device="cuda").bfloat16()

        def fwd():
            with torch.no_grad():
                bi, add = hc(H)
                return add(bo)

        def step():
            H.grad = None
            bo.grad = None
            for p in params:
                p.grad = None
            bi, add = hc(H)
            torch.autograd.backward([add(bo), bi], [dHn, dbi])

        rec = {}
        for name, fn, units in (("fwd_nograd", fwd, 18), ("fwd_bwd", step, 42)):
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(3):
                    fn()
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                fn()
            for _ in range(5):
                g.replay()
            torch.cuda.synchronize()
            ts = []
            for _ in range(reps):
                t0 = time.perf_counter()
                for _ in range(calls):
                    g.replay()
                torch.cuda.synchronize()
                ts.append((time.perf_counter() - t0) / calls * 1e6)
            us = statistics.median(ts)
            nbytes = units * D * 2 * B * S
            rec[name] = {"us": round(us, 1), "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
            del g
        out[f"B={B} S={S}"] = rec
    return out


OPS_GROUPS = ("sinkhorn", "stream", "dynw_rows", "dynw_bf16", "dynw_other")


def _ops_leg(n: int = 20, warm: int = 3, groups=OPS_GROUPS) -> dict:
    """Each low-level op alone, timed with HIP events on torch's current stream
    (the stream the kernels run on): time per call (the median of three blocks of
    ``n`` calls, each block's mean, so that a stretch of lowered clocks on the box
    moves one block, not the figure) and the fraction of 8 TB/s its algorithmic
    bytes reach.  Inputs are resident before timing; gradient calls use
    torch.autograd.grad, so nothing accumulates between calls.  ``groups`` picks
    from OPS_GROUPS: config-2 Sinkhorn, the stream ops at config-3 size, dynamic
    weights at R = 4, at R = K = 16384 bf16, and at R = K = 16384 fp16 / fp32."""
    import torch

    import mhc
    from mhc import _backward as KB
    from mhc import _kernels as K

    dev = "cuda"
    g = torch.Generator(device=dev)
    g.manual_seed(0)

    def timed(fn, calls=n, blocks=3):
        for _ in range(warm):
            fn()
        torch.cuda.synchronize()
        per_block = []
        for _ in range(blocks):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            # a bounded spin kernel ahead of the first event keeps the GPU busy while the host
            # queues the first calls, so the host's start-up latency stays out of the interval
            torch.cuda._sleep(1 << 20)
            a.record()
            for _ in range(calls):
                fn()
            b.record()
            torch.cuda.synchronize()
            per_block.append(a.elapsed_time(b) / calls * 1e3)  # us
        return statistics.median(per_block)

    out = {}

    def rec(name, us, nbytes):
        out[name] = {"us": round(us, 1), "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}

    if "sinkhorn" in groups:
        # config 2: Sinkhorn over 2^20 fp32 matrices (fwd reads M, writes P; bwd reads M, dP, writes dM)
        M = torch.exp(torch.randn((1 << 20, 4, 4), generator=g, device=dev))
        dP = torch.randn((1 << 20, 4, 4), generator=g, device=dev)
        rec("sinkhorn_fwd config2", timed(lambda: K.sinkhorn_forward(M, 20, 1e-8)), 2 * M.numel() * 4)
        rec("sinkhorn_bwd config2", timed(lambda: KB.sinkhorn_backward(M, dP, 20, 1e-8)), 3 * M.numel() * 4)
        del M, dP
    B, S, D = 4, 4096, 4096
    e, T = 2, B * S
    if "stream" in groups:
        _stream_ops(g, B, S, D, timed, rec)
    # fused dynamic weights: R = B rows (the module's use) and R = tokens rows (bf16, MFMA path)
    phi = torch.randn((4 * D, 24), generator=g, device=dev) * 0.02
    bias = torch.randn(24, generator=g, device=dev)
    al = [torch.tensor([0.1], device=dev) for _ in range(3)]
    if "dynw_rows" in groups:
        x4 = torch.randn((4, 4 * D), generator=g, device=dev)
        rec("dynamic_weights_fwd R=4 K=16384 f32",
            timed(lambda: K.fused_dynamic_weights_forward(x4, phi, bias, *al)), 4 * 4 * D * 4)
    phl = phi.clone().requires_grad_(True)
    gs = [torch.randn((T, 4), generator=g, device=dev), torch.randn((T, 4), generator=g, device=dev),
          torch.randn((T, 4, 4), generator=g, device=dev)]
    # bf16 rows, then the same op on fp16 and fp32 rows (MFMA kernels: fp16 forward on the f16
    # MFMA, the rest with x split into bf16 parts in registers); x read by the forward, x read
    # and grad_x written by the backward
    dts = ((torch.bfloat16, "bf16"),) if "dynw_bf16" in groups else ()
    if "dynw_other" in groups:
        dts += ((torch.float16, "f16"), (torch.float32, "f32"))
    for dt, tag in dts:
        xd = torch.randn((T, 4 * D), generator=g, device=dev).to(dt)
        nb = T * 4 * D * xd.element_size()
        rec(f"dynamic_weights_fwd R=16384 K=16384 {tag}",
            timed(lambda: K.fused_dynamic_weights_forward(xd, phi, bias, *al)), nb)
        xdl = xd.clone().requires_grad_(True)

        def fwd_bwd_d():
            o = mhc.fused_dynamic_weights(xdl, phl, bias, *al)
            torch.autograd.grad(o, [xdl, phl], gs)

        rec(f"dynamic_weights_fwd+bwd R=16384 K=16384 {tag}", timed(fwd_bwd_d), 3 * nb)
        del xd, xdl
    return out


def _stream_ops(g, B, S, D, timed, rec) -> None:
    """The stream ops at one layout (bf16), for _ops_leg."""
    import torch

    from mhc import _backward as KB
    from mhc import _kernels as K

    dev = "cuda"
    e, T = 2, B * S
    H = torch.randn((B, S, 4, D), generator=g, device=dev).bfloat16()
    pre = torch.softmax(torch.randn((B, 4), generator=g, device=dev), -1)
    res = K.sinkhorn_forward(torch.randn((B, 4, 4), generator=g, device=dev), 20, 1e-8)
    post = torch.rand((B, 4), generator=g, device=dev) * 2
    bo = torch.randn((B, S, D), generator=g, device=dev).bfloat16()
    rec("stream_mix_fwd config3", timed(lambda: K.stream_mix_forward(H, pre, res)), 9 * D * e * T)
    bi, hr = K.stream_mix_forward(H, pre, res)
    rec("add_residual_fwd config3", timed(lambda: K.add_residual_forward(hr, bo, post)), 9 * D * e * T)
    dhn = torch.randn((B, S, 4, D), generator=g, device=dev).bfloat16()
    rec("add_residual_bwd config3", timed(lambda: KB.add_residual_backward(dhn, bo, post)), 6 * D * e * T)
    rec("stream_mix_bwd config3", timed(lambda: KB.stream_mix_backward(bi, dhn, H, pre, res)), 13 * D * e * T)
    rec("mean_pool config3", timed(lambda: K.mean_pool(H)), 4 * D * e * T)
    rec("stream_expand config3", timed(lambda: K.stream_expand(bo)), 5 * D * e * T)
    rec("stream_collapse config3", timed(lambda: K.stream_collapse(H, 0.25)), 5 * D * e * T)


# The reference's published table (README.md:183-202): NVIDIA H100 80GB HBM3, batch=16, seq=2048,
# dim=4096, fp16, made by benchmarks/benchmark.py.  Times in ms, memory in MB.
README_PUBLISHED = {
    "sinkhorn_20iter": {"pytorch_ms": 0.74, "triton_ms": 0.47},
    "stream_mix": {"pytorch_ms": 8.53, "triton_ms": 1.00},
    "add_residual": {"pytorch_ms": 2.57, "triton_ms": 0.89},
    "dynamic_weights": {"pytorch_ms": 0.90, "triton_ms": 0.11},
    "full_forward_backward": {"pytorch_ms": 85.00, "triton_ms": 13.66},
    "peak_memory_sinkhorn_backward": {"pytorch_mb": 120.0, "triton_mb": 68.0},
    "peak_memory_full_forward_backward": {"pytorch_mb": 8003.6, "triton_mb": 6162.8},
}


def _readme_leg(batch: int = 16, seq: int = 2048, dim: int = 4096) -> dict:
    """The reference's benchmark table on this build, one op at a time, the way
    benchmarks/benchmark.py measures it: 10 warm-up calls, then the mean wall time of 100
    calls between two device synchronisations (time.perf_counter), on fp16 inputs drawn
    as the script draws them (:53-138, :141-180).  The same workloads also run through
    the package's pure-PyTorch baselines (the reference's `*_torch` path) on this GPU, and
    peak memory is measured as the script does (:184-200)."""
    import torch

    import mhc

    dev = "cuda"
    torch.manual_seed(0)

    def wall_ms(fn, warmup=10, repeats=100):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        t = time.perf_counter()
        for _ in range(repeats):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t) / repeats * 1e3

    def peak_mb(fn, warmup=3):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats()
        fn()
        torch.cuda.synchronize()
        return torch.cuda.max_memory_allocated() / (1024 * 1024)

    out = {}

    def rec(name, ours, torch_path, unit="ms"):
        pub = README_PUBLISHED[name]
        key = "triton_" + unit
        out[name] = {f"ours_{unit}": round(ours, 4), f"torch_baseline_mi355x_{unit}": round(torch_path, 4),
                     f"published_h100_triton_{unit}": pub[key],
                     f"published_h100_pytorch_{unit}": pub["pytorch_" + unit],
                     "published_triton_over_ours": round(pub[key] / ours, 2)}

    half = torch.float16

    # Each workload lives in its own function, as in the script, so that nothing from
    # another one is allocated while it is measured.
    def sinkhorn():  # (:53-64), batch*seq matrices
        M = torch.randn(batch * seq, 4, 4, device=dev, dtype=half)
        rec("sinkhorn_20iter", wall_ms(lambda: mhc.sinkhorn_knopp(M, num_iters=20)),
            wall_ms(lambda: mhc.sinkhorn_knopp_torch(M, num_iters=20)))

    def stream_mix():  # (:67-83)
        H = torch.randn(batch, seq, 4, dim, device=dev, dtype=half)
        H_pre = torch.softmax(torch.randn(batch, 4, device=dev, dtype=half), dim=-1)
        H_res = mhc.sinkhorn_knopp(torch.randn(batch, 4, 4, device=dev, dtype=half), num_iters=20)
        rec("stream_mix", wall_ms(lambda: mhc.fused_stream_mix(H, H_pre, H_res)),
            wall_ms(lambda: mhc.fused_stream_mix_torch(H, H_pre, H_res)))

    def add_residual():  # (:86-106)
        H_residual = torch.randn(batch, seq, 4, dim, device=dev, dtype=half)
        bo = torch.randn(batch, seq, dim, device=dev, dtype=half)
        H_post = torch.softmax(torch.randn(batch, 4, device=dev, dtype=half), dim=-1)
        rec("add_residual", wall_ms(lambda: mhc.fused_add_residual(H_residual, bo, H_post)),
            wall_ms(lambda: mhc.fused_add_residual_torch(H_residual, bo, H_post)))

    def dynamic_weights():  # (:109-138), x [batch, 4*dim] fp32
        x = torch.randn(batch, 4 * dim, device=dev)
        phi = torch.randn(4 * dim, 24, device=dev) * 0.01
        bias = torch.randn(24, device=dev)
        al = [torch.tensor(0.1, device=dev) for _ in range(3)]
        rec("dynamic_weights", wall_ms(lambda: mhc.fused_dynamic_weights(x, phi, bias, *al)),
            wall_ms(lambda: mhc.fused_dynamic_weights_torch(x, phi, bias, *al)))

    def full_layer(measure):  # (:141-180 and :226-260), fp16 module
        hc = mhc.HyperConnection(dim=dim, num_streams=4, dynamic=True).to(dev).half()
        hc_t = mhc.HyperConnectionTorch(dim=dim, num_streams=4, dynamic=True).to(dev).half()
        hc_t.load_state_dict(hc.state_dict())
        H = torch.randn(batch, seq, 4, dim, device=dev, dtype=half, requires_grad=True)

        def fwd_bwd(module):
            def run():
                H_in = H.detach().requires_grad_(True)
                bi, add_residual = module(H_in)
                H_new = add_residual(bi * 0.5)
                H_new.sum().backward()
                return H_in.grad
            return run

        if measure == "time":
            rec("full_forward_backward", wall_ms(fwd_bwd(hc)), wall_ms(fwd_bwd(hc_t), warmup=2, repeats=10))
        else:
            ours = peak_mb(fwd_bwd(hc))
            rec("peak_memory_full_forward_backward", ours, peak_mb(fwd_bwd(hc_t)), unit="mb")

    def sinkhorn_memory():  # (:203-223)
        M = torch.randn(batch * seq, 4, 4, device=dev, dtype=half, requires_grad=True)

        def sk_bwd(fn):
            def run():
                M_in = M.detach().requires_grad_(True)
                fn(M_in, num_iters=20).sum().backward()
                return M_in.grad
            return run

        ours = peak_mb(sk_bwd(mhc.sinkhorn_knopp))
        rec("peak_memory_sinkhorn_backward", ours, peak_mb(sk_bwd(mhc.sinkhorn_knopp_torch)), unit="mb")

    # Memory first, ours before the PyTorch path: the latter's matmuls leave a BLAS workspace
    # allocated through the caching allocator that later peaks would include.
    for leg in (sinkhorn_memory, lambda: full_layer("memory"), sinkhorn, stream_mix, add_residual,
                dynamic_weights, lambda: full_layer("time")):
        leg()
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return out


def _build_inputs(cfg, dev):
    import torch

    import mhc

    B, S, D = cfg["B"], cfg["S"], cfg["D"]
    dt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[cfg["dtype"]]
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    hc = mhc.HyperConnection(D, dynamic=cfg["dynamic"]).to(dev)
    H = torch.randn((B, S, 4, D), generator=g, device=dev, dtype=torch.float32).to(dt)
    with torch.no_grad():
        if cfg["dynamic"]:
            hc.phi.copy_(torch.randn((24, 4 * D), generator=g, device=dev).T * 0.02)
        else:
            hc.H_res_base.copy_(torch.randn((4, 4), generator=g, device=dev))
    bo = torch.randn((B, S, D), generator=g, device=dev, dtype=torch.float32).to(dt)
    dH_new = torch.randn((B, S, 4, D), generator=g, device=dev, dtype=torch.float32).to(dt)
    d_bi = torch.randn((B, S, D), generator=g, device=dev, dtype=torch.float32).to(dt)
    H.requires_grad_(True)
    bo.requires_grad_(True)
    return hc, H, bo, dH_new, d_bi


def _gpu_leg(cfg, steps, warmup):
    import torch

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    hc, H, bo, dH_new, d_bi = _build_inputs(cfg, dev)
    params = list(hc.parameters())
    stream = torch.cuda.current_stream(dev)

    def step(ev=None):
        H.grad = None
        bo.grad = None
        for p in params:
            p.grad = None
        bi, add = hc(H)
        if ev is not None:
            ev[0].record(stream)
        H_new = add(bo)  # one kernel: H_new = H_res @ H + H_post * bo
        if ev is not None:
            ev[1].record(stream)
        torch.autograd.backward([H_new, bi], [dH_new, d_bi])

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()

    # Forward-only rate (no autograd graph), same inputs.
    with torch.no_grad():
        for _ in range(3):
            bi, add = hc(H)
            add(bo)
        torch.cuda.synchronize()
        f0 = torch.cuda.Event(enable_timing=True)
        f1 = torch.cuda.Event(enable_timing=True)
        f0.record(stream)
        for _ in range(steps):
            bi, add = hc(H)
            add(bo)
        f1.record(stream)
        torch.cuda.synchronize()
    fwd_ms = f0.elapsed_time(f1) / steps
    del bi, add

    # The dominant kernel is bracketed by HIP events on every KERNEL_SAMPLE_EVERY-th timed step.
    # Each recorded event is a marker packet that drains the queue: an event pair leaves the GPU
    # idle for about 11 us around the kernel (two ~5.7 us dispatch gaps in a kernel trace), time
    # that belongs to the measurement, not to the step.
    sampled = set(range(0, steps, KERNEL_SAMPLE_EVERY))
    kev = {i: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for i in sampled}
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t0.record(stream)
    for i in range(steps):
        step(kev.get(i))
    t1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms = t0.elapsed_time(t1) / steps
    add_ms = sum(a.elapsed_time(b) for a, b in kev.values()) / len(kev)
    return dict(ms=ms, wall_ms=wall * 1e3 / steps, fwd_ms=fwd_ms, add_ms=add_ms, add_samples=len(kev),
                elem=H.element_size(), device=torch.cuda.get_device_name(dev))


def _workload_summary(name, cfg, r) -> dict:
    """The figures of one workload's GPU leg, in the units of the main line."""
    B, S, D = cfg["B"], cfg["S"], cfg["D"]
    T, e = B * S, r["elem"]
    fu, bu = ALGO_UNITS[cfg["dynamic"]]
    add_gbs = 9 * D * e * T / (r["add_ms"] * 1e-3) / 1e9
    return {
        "workload": f"{name}: HyperConnection layer fwd+bwd, dim={D}, num_streams=4, "
                    f"{'dynamic fused' if cfg['dynamic'] else 'static'} weights, sinkhorn_iters=20",
        "B": B, "S": S, "D": D, "dtype": cfg["dtype"],
        "ms_per_step": round(r["ms"], 5),
        "tokens_per_s": round(T / (r["ms"] * 1e-3), 1),
        "layer_roofline": {"algorithmic_bytes_per_step": (fu + bu) * D * e * T,
                           "frac": round((fu + bu) * D * e * T / (r["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
        "fwd_only": {"ms_per_step": round(r["fwd_ms"], 5), "tokens_per_s": round(T / (r["fwd_ms"] * 1e-3), 1),
                     "frac": round(fu * D * e * T / (r["fwd_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
        "closure_forward": {"us": round(r["add_ms"] * 1e3, 1), "achieved_GBps": round(add_gbs, 1),
                            "frac": round(add_gbs / HBM_PEAK_GBS, 4), "timed_launches": r["add_samples"],
                            "traffic": MEASURED_TRAFFIC.get(name), "traffic_measured_at": TRAFFIC_COMMIT},
    }


def _cpu_leg(cfg, reps: int = 3, seq: int | None = None):
    """The reference's pure-PyTorch layer (restated in oracle/torch_path.py), on the host
    cores, at the workload's own shape (B, S, D): forward, and forward + autograd backward,
    fp32-upcast (the reference's own torch path raises on bf16 H with fp32 weights,
    _torch_baseline.py:136,141).  One warm-up run, then the median of `reps` runs, as the
    reference's benchmark times its large cases.  `seq` shortens the sequence (tests only)."""
    import torch

    from oracle import torch_path

    B, D = cfg["B"], cfg["D"]
    S = cfg["S"] if seq is None else seq
    g = torch.Generator()
    g.manual_seed(0)
    p = {
        "H_pre_base": torch.nn.functional.one_hot(torch.tensor(0), 4).float(),
        "H_post_base": torch.ones(4),
        "H_res_base": torch.eye(4) if cfg["dynamic"] else torch.randn((4, 4), generator=g),
    }
    if cfg["dynamic"]:
        p["phi"] = torch.randn((24, 4 * D), generator=g).T.contiguous() * 0.02
        for k in ("alpha_pre", "alpha_post", "alpha_res"):
            p[k] = torch.tensor([0.1])
    H = torch.randn((B, S, 4, D), generator=g)
    bo = torch.randn((B, S, D), generator=g)
    dHn = torch.randn((B, S, 4, D), generator=g)
    dbi = torch.randn((B, S, D), generator=g)

    def fwd_bwd():
        torch_path.layer_grads(p, H, bo, dHn, dbi, dynamic=cfg["dynamic"], fused=True)

    def fwd():
        with torch.no_grad():
            torch_path.layer_forward(p, H, bo, dynamic=cfg["dynamic"], fused=True)

    def median_s(fn, label):
        t = time.perf_counter()
        fn()  # warm-up (first touch of the working set)
        _log(f"bench: cpu {label} warm-up {time.perf_counter() - t:.2f} s")
        runs = []
        for i in range(reps):
            t = time.perf_counter()
            fn()
            runs.append(time.perf_counter() - t)
            _log(f"bench: cpu {label} run {i + 1}/{reps} {runs[-1]:.2f} s")
        return statistics.median(runs), runs

    t_fb, runs_fb = median_s(fwd_bwd, "fwd+bwd")
    t_f, _ = median_s(fwd, "fwd")
    T = B * S
    return {
        "value": round(T / t_fb, 1),
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"the whole workload: torch CPU fp32 restatement of the reference's pure-PyTorch layer, "
                   f"B={B} S={S} D={D} ({'dynamic fused' if cfg['dynamic'] else 'static'}), fwd + autograd bwd, "
                   f"median of {reps} runs after 1 warm-up"),
        "ms_per_step": round(t_fb * 1e3, 1),
        "runs_s": [round(r, 3) for r in runs_fb],
        "fwd_only_tokens_per_s": round(T / t_f, 1),
        "torch_version": torch.__version__,
        "host_cpus": os.cpu_count(),
        "host_cpu_model": _cpu_model(),
    }


def _cpu_model() -> str | None:
    """The host CPU's model name from /proc/cpuinfo (None where that file is absent)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def main() -> int:
    args = _parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}); "
              "the mHC layer path has no multi-GPU leg here", file=sys.stderr, flush=True)
        return 2
    if args.steps < 1 or args.warmup < 0:
        print("bench.py: --steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        return 1
    if args.calibrate_copy:
        return _calibrate_copy()
    if args.dynw_ceiling:
        from mhc import _lib

        _lib.load()
        print(json.dumps({"dynw_ceiling": _dynw_ceiling(), "unit": "us per launch", "peak_GBps": HBM_PEAK_GBS,
                          "device": torch.cuda.get_device_name(0)}), flush=True)
        return 0
    if args.stream_ceiling:
        cfg = WORKLOADS[args.workload]
        tokens, row_bytes = cfg["B"] * cfg["S"], cfg["D"] * (2 if cfg["dtype"] in ("bf16", "fp16") else 4)
        print(json.dumps({"stream_ceiling": _stream_ceiling(tokens, row_bytes), "unit": "us per launch",
                          "peak_GBps": HBM_PEAK_GBS, "workload": args.workload,
                          "layout": f"{tokens} tokens x {row_bytes}-byte rows per array row",
                          "caps": "cap0 = no occupancy cap, capN = at most N workgroups per CU",
                          "device": torch.cuda.get_device_name(0)}), flush=True)
        return 0
    from mhc import _lib

    _lib.load()  # fails loudly when the HIP library is not built
    if args.ops:
        print(json.dumps({"ops": _ops_leg(), "unit": "us per call", "peak_GBps": HBM_PEAK_GBS,
                          "device": torch.cuda.get_device_name(0)}), flush=True)
        return 0
    if args.decode:
        print(json.dumps({"decode": _decode_leg(), "unit": "us per replayed step", "dim": 4096, "dtype": "bf16",
                          "layer": "HyperConnection(dynamic=True), phi ~ N(0, 0.02)",
                          "device": torch.cuda.get_device_name(0)}), flush=True)
        return 0
    if args.readme:
        print(json.dumps({"readme_table": _readme_leg(),
                          "config": {"batch": 16, "seq": 2048, "dim": 4096, "dtype": "fp16"},
                          "method": "benchmarks/benchmark.py: mean wall time of 100 calls after 10 "
                                    "warm-up (PyTorch full fwd+bwd: 10 after 2), device-synchronised",
                          "published_hardware": "NVIDIA H100 80GB HBM3 (README.md:185)",
                          "device": torch.cuda.get_device_name(0)}), flush=True)
        return 0

    cfg = WORKLOADS[args.workload]
    B, S, D = cfg["B"], cfg["S"], cfg["D"]
    T = B * S
    _log(f"bench: {args.workload} B={B} S={S} D={D} {cfg['dtype']} warmup={args.warmup} steps={args.steps}")
    r = _gpu_leg(cfg, args.steps, args.warmup)
    e = r["elem"]
    fu, bu = ALGO_UNITS[cfg["dynamic"]]
    step_bytes = (fu + bu) * D * e * T
    fwd_bytes = fu * D * e * T
    add_bytes = 9 * D * e * T  # H_new kernel: reads H (4) + bo (1), writes H_new (4)
    _log(f"bench: gpu {r['ms']:.4f} ms/step (wall {r['wall_ms']:.4f}), fwd {r['fwd_ms']:.4f} ms, "
         f"H_new kernel {r['add_ms'] * 1e3:.1f} us")

    # Configs 4 and 5 ride along with the default config-3 run (GPU legs only, about a second each).
    workloads = {}
    if args.workload == "config3" and not args.no_workloads:
        for name in ("config4", "config5"):
            wr = _gpu_leg(WORKLOADS[name], args.steps, args.warmup)
            workloads[name] = _workload_summary(name, WORKLOADS[name], wr)
            _log(f"bench: {name} {wr['ms']:.4f} ms/step, layer {workloads[name]['layer_roofline']['frac']:.4f} of "
                 f"8 TB/s, H_new kernel {wr['add_ms'] * 1e3:.1f} us")
        # config 2 (Sinkhorn over 2^20 matrices) and the dynamic-weights op at R = tokens (the
        # MFMA kernels), as `--ops` times them: well under a second of GPU time
        ops = _ops_leg(groups=("sinkhorn", "dynw_bf16"))
        workloads["ops"] = {"unit": "us per call (median of three blocks of 20), hbm_frac of 8 TB/s", **ops}
        for k, v in ops.items():
            _log(f"bench: {k} {v['us']} us, {v['hbm_frac']:.4f} of 8 TB/s")

    cpu = None
    if args.cpu_reps > 0:
        _log("bench: cpu baseline ...")
        cpu = _cpu_leg(cfg, args.cpu_reps)
        _log(f"bench: cpu {cpu['value']} tokens/s on {cpu['cores']} threads")

    add_gbs = add_bytes / (r["add_ms"] * 1e-3) / 1e9
    step_gbs = step_bytes / (r["ms"] * 1e-3) / 1e9
    out = {
        "metric": METRIC,
        "value": round(T / (r["ms"] * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": "synthetic (N(0,1) inputs, phi ~ N(0, 0.02), seed 0; generated on the GPU)",
        "config": {
            "workload": f"{args.workload}: HyperConnection layer fwd+bwd, dim={D}, num_streams=4, "
                        f"{'dynamic fused' if cfg['dynamic'] else 'static'} weights, sinkhorn_iters=20",
            "B": B, "S": S, "D": D, "tokens_per_step": T, "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "H_new = H_res @ H + H_post * bo (mix_fwd_kernel, closure forward)",
            "achieved": round(add_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(add_gbs / HBM_PEAK_GBS, 4),
            "traffic": MEASURED_TRAFFIC.get(args.workload),
            "traffic_measured_at": TRAFFIC_COMMIT,
            "timed_launches": r["add_samples"],
            "mix_ceiling_frac": STREAM_CEILING_5_4.get(args.workload),
            "frac_of_mix_ceiling": (round(add_gbs / HBM_PEAK_GBS / STREAM_CEILING_5_4[args.workload], 4)
                                    if STREAM_CEILING_5_4.get(args.workload) else None),
        },
        "layer_roofline": {
            "algorithmic_bytes_per_step": step_bytes,
            "achieved_GBps": round(step_gbs, 1),
            "frac": round(step_gbs / HBM_PEAK_GBS, 4),
        },
        "fwd_only": {
            "ms_per_step": round(r["fwd_ms"], 5),
            "tokens_per_s": round(T / (r["fwd_ms"] * 1e-3), 1),
            "frac": round(fwd_bytes / (r["fwd_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        },
        "wall_ms_per_step": round(r["wall_ms"], 5),
        "compute_dtype": "fp32 arithmetic on bf16/fp16 storage",
        "device": r["device"],
        "cpu_baseline": cpu,
    }
    if workloads:
        out["workloads"] = workloads
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
