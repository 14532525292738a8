"""The dynamic layer on both sides of each of its size thresholds, against the float64 oracle.

The layer picks its kernels from B, S and D (csrc/layer.hip, csrc/dynamic_weights.hip):

* from 64 batches (kLayerBulkRows) the weights backward runs on the MFMA kernel in row chunks;
* at S = 1 from 64 batches (kLayerBulkProjRowsS1) the projection runs on the MFMA kernel over
  H's own rows, and no pooled rows are formed;
* for S > 1 from 64 batches, once B * D reaches 2^19 (kLayerBulkProjElems), the mean-pool runs
  without the projection and the pooled rows are projected on the MFMA kernel;
* the mean-pool takes one launch for S <= 8 and the column-sum + reduce pair beyond.

Each case runs a training step (every gradient) and a no-grad forward, whose outputs must be the
same bits as the training forward's.  Dynamic fused weights, phi ~ N(0, 0.02).
"""

import pytest
import torch

from test_gpu_module import check_layer, make_case

pytestmark = pytest.mark.gpu

CASES = [
    # S = 1: the MFMA projection on H's rows and the row-chunk backward start at 64 batches
    (63, 1, 64, torch.bfloat16), (64, 1, 64, torch.bfloat16), (65, 1, 64, torch.bfloat16),
    (63, 1, 128, torch.float16), (64, 1, 128, torch.float16),
    (63, 1, 32, torch.float32), (64, 1, 32, torch.float32),
    # S > 1: B * D = 2^19 at B = 64, D = 8192 (pooled-row projection); one batch fewer, or a
    # D eight columns narrower, keeps the projection folded into the mean-pool's reduce
    (63, 2, 8192, torch.bfloat16), (64, 2, 8192, torch.bfloat16), (64, 2, 8184, torch.bfloat16),
    # the single-launch mean-pool (S <= 8) against the column-sum + reduce pair (S = 9), with
    # the pooled-row projection
    (64, 8, 8192, torch.bfloat16), (64, 9, 8192, torch.bfloat16),
    # and with the projection folded (B * D below 2^19)
    (64, 8, 64, torch.bfloat16), (64, 9, 64, torch.bfloat16),
]


@pytest.mark.parametrize("B,S,D,dtype", CASES)
def test_layer_on_both_sides_of_its_thresholds(B, S, D, dtype):
    print(f"case B={B} S={S} D={D} {dtype}", flush=True)
    hc, H, bo, dHn, dbi = make_case(B, S, D, dtype, phi_std=0.02)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    check_layer(hc, H, bo, dHn, dbi, tol, 1e-4 if dtype == torch.float32 else 2e-2, 1e-4)
    bi, add = hc(H.clone().requires_grad_(True))
    Hn = add(bo)
    with torch.no_grad():
        bi0, add0 = hc(H)
        Hn0 = add0(bo)
    assert torch.equal(bi0, bi.detach()) and torch.equal(Hn0, Hn.detach())
