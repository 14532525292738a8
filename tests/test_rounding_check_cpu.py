"""The once-rounded check of test_gpu_rounding.py (helpers.rounded_once_stats), pinned on
the CPU: an fp32 evaluation rounded to nearest-even passes it, while truncation instead of
rounding and weights rounded to the half format before use fail it."""

import pytest
import torch

from helpers import MISMATCH, rounded_once_stats


def _case(dtype, n=1 << 18, seed=0):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn((4, n), generator=g, dtype=torch.float64).to(dtype)
    w = torch.rand(4, generator=g, dtype=torch.float64).float()
    h64, w64 = h.double(), w.double()
    ref64 = (w64[:, None] * h64).sum(0)
    absterm = (w64[:, None].abs() * h64.abs()).sum(0)
    return h, w, ref64, absterm


def _truncate(x32, dtype):
    """fp32 -> bf16 / fp16 by dropping the low bits (round toward zero)."""
    if dtype == torch.bfloat16:
        bits = x32.view(torch.int32) & ~0xFFFF
        return bits.view(torch.float32).to(dtype)
    r = x32.to(dtype)  # fp16: step the magnitude back one ulp where nearest-even rounded away from zero
    bits = r.view(torch.int16).to(torch.int32) & 0xFFFF
    back = ((bits & 0x7FFF) - 1) | (bits & 0x8000)
    away = r.float().abs() > x32.abs()
    out = torch.where(away, back, bits)
    return torch.where(out >= 0x8000, out - 0x10000, out).to(torch.int16).view(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fp32_then_round_to_nearest_even_passes(dtype):
    h, w, ref64, absterm = _case(dtype)
    got = (w[:, None] * h.float()).sum(0).to(dtype)
    worst, frac = rounded_once_stats(got, ref64, absterm)
    assert worst <= 1.0 and frac <= MISMATCH[str(dtype)[6:]]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_truncation_fails(dtype):
    h, w, ref64, absterm = _case(dtype)
    got = _truncate((w[:, None] * h.float()).sum(0), dtype)
    worst, frac = rounded_once_stats(got, ref64, absterm)
    assert frac > 0.2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_weights_rounded_to_half_first_fail(dtype):
    h, w, ref64, absterm = _case(dtype)
    got = (w.to(dtype).float()[:, None] * h.float()).sum(0).to(dtype)
    worst, frac = rounded_once_stats(got, ref64, absterm)
    assert frac > 10 * MISMATCH[str(dtype)[6:]]
