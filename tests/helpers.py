"""Small helpers shared by the test modules."""

import numpy as np


def rel_err(a, b) -> float:
    """Normwise relative error max|a - b| / max(max|b|, 1e-30), one number per tensor."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    if a.shape != b.shape:
        raise AssertionError(f"shape mismatch {a.shape} vs {b.shape}")
    if b.size == 0:
        return 0.0
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def to_np(t):
    """torch tensor (any device / dtype) -> float64 numpy array."""
    import torch

    return t.detach().to("cpu", torch.float64).numpy()


# Significand bits (with the implicit one) and the smallest subnormal of the half formats.
_HALF = {"bfloat16": (8, 2.0 ** -133), "float16": (11, 2.0 ** -24)}


def rounded_once_stats(got, ref64, absterm64):
    """Compare a bf16 / fp16 kernel output with the float64 value of the same expression.

    ``ref64`` is the expression evaluated in float64 from the kernel's own inputs and fp32
    weights; ``absterm64`` is the sum of the absolute values of its terms (it bounds the
    error of an fp32 evaluation: a few 2^-24 times it).  A kernel that computes in fp32 and
    rounds once to nearest-even lands within one unit in the last place of the once-rounded
    reference everywhere, and on exactly the same bits except where the fp32 evaluation
    error straddles a rounding boundary: a small fraction of the elements.  Truncating
    instead of rounding, or weights rounded to the half format first, moves a large
    fraction of the elements.

    Returns (worst |got - ref| / allowed, fraction of elements whose bits differ); the
    caller asserts the first <= 1 and the second below the format's threshold."""
    import torch

    nbits, tiny = _HALF[str(got.dtype).replace("torch.", "")]
    ref = ref64.to(got.dtype)
    a = ref.double().abs()
    ulp = torch.pow(2.0, torch.floor(torch.log2(a.clamp_min(tiny))) - (nbits - 1)).clamp_min(tiny)
    allowed = ulp + 8 * 2.0 ** -24 * absterm64
    got = got.detach()
    worst = float(((got.double() - ref.double()).abs() / allowed).max()) if got.numel() else 0.0
    diff = (got.view(torch.int16) != ref.view(torch.int16)).double().mean() if got.numel() else 0.0
    return worst, float(diff)


# Largest fraction of elements allowed to differ in bits from the once-rounded float64 value.
MISMATCH = {"bfloat16": 1e-3, "float16": 5e-3}


def assert_rounded_once(got, ref64, absterm64, what=""):
    worst, frac = rounded_once_stats(got, ref64, absterm64)
    print(f"rounded-once {what} {got.dtype}: worst/allowed={worst:.3f} bit-mismatch={frac:.2e}", flush=True)
    assert worst <= 1.0, (what, worst, frac)
    assert frac <= MISMATCH[str(got.dtype).replace("torch.", "")], (what, worst, frac)
