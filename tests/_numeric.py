"""Tolerances and comparison helpers (after the reference's tests/_numeric.py:24-68).

The north-star bar for values is max relative error <= 2e-2 against the fp32
oracle, relative to the expected tensor's global max magnitude.
"""

import torch

LAYOUT_RTOL = 0
LAYOUT_ATOL = 0
REL_TOL = 2e-2          # max |a - b| / max |b|
OUTPUT_RTOL = 4e-2      # reference forward output tolerance (tests/_numeric.py:30-31)
OUTPUT_ATOL = 4e-2
GRAD_RTOL = 2e-2        # reference gradient tolerance (tests/_numeric.py:33-34)
GRAD_ATOL = 1e-2


def max_rel(actual, expected) -> float:
    a = actual.detach().float().cpu()
    b = expected.detach().float().cpu()
    if b.numel() == 0:
        return 0.0
    return float((a - b).abs().max()) / (float(b.abs().max()) + 1e-12)


def assert_rel(actual, expected, tol=REL_TOL, name=""):
    assert tuple(actual.shape) == tuple(expected.shape), f"{name}: shape {tuple(actual.shape)} != {tuple(expected.shape)}"
    a = actual.detach().float().cpu()
    assert torch.isfinite(a).all(), f"{name}: non-finite values"
    r = max_rel(actual, expected)
    assert r <= tol, f"{name}: max relative error {r:.3e} > {tol:.1e}"


def cmp_grad(tri, gold, rtol=GRAD_RTOL, atol=GRAD_ATOL):
    """Reference-style check: count elements with |d| > atol + rtol * max|gold|."""
    tri = tri.float().cpu()
    gold = gold.float().cpu()
    d = (tri - gold).abs()
    gmax = float(gold.abs().max()) if gold.numel() else 0.0
    return int((d > atol + rtol * gmax).sum())
