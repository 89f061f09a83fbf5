"""Check of a saved FC1 output against the oracle's, within one rounding step.

The build and the oracle form FC1 as fp32 sums over the hidden dimension in
different orders, then round to the saved format; the saved values can
therefore differ by one rounding step of that format, and no more.
"""

import torch

from oracle import moe_oracle as O


def bf16_ulp(v: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 values at |v| (8 significant bits); the subnormal
    floor is irrelevant at these magnitudes."""
    e = torch.floor(torch.log2(v.abs().clamp_min(2.0 ** -126)))
    return torch.exp2(e - 7)


def e4m3_magnitude_index(q: torch.Tensor) -> torch.Tensor:
    """Signed position of each E4M3 code on the number line: adjacent
    representable values differ by one (the code's low 7 bits order the
    magnitudes)."""
    b = q.view(torch.uint8).to(torch.int32)
    mag = b & 0x7F
    return torch.where(b & 0x80 != 0, -mag, mag)


def check_saved_fc1(saved, st, m, fmt):
    """(i): the saved FC1 output is the oracle's within one rounding step."""
    if fmt == "fp8":
        s_gpu, s_ref = saved["fc1_output_scale"][:m].float().cpu(), st["fc1_output_scale"].float()
        # scale = amax / 448 with amax a bf16 value: one ulp of amax apart at most
        amax = s_ref * O.FP8_MAX
        assert torch.all((s_gpu - s_ref).abs() <= bf16_ulp(amax) / O.FP8_MAX * 1.0001), \
            "fp8 scale moved by more than one bf16 ulp of the group amax"
        moved = s_gpu != s_ref
        step = (e4m3_magnitude_index(saved["fc1_output"][:m].cpu()) - e4m3_magnitude_index(st["fc1_output"])).abs()
        assert int(step.max()) <= 1, f"fp8 code differs by {int(step.max())} steps"
        return moved
    a = saved["fc1_output"][:m].float().cpu()
    b = st["fc1_output"].float()
    d = (a - b).abs()
    # one bf16 ulp; plus the fp32 sum's own error where FC1 cancels to a
    # value far below its terms (|gu| < 2^-10 of the row's max)
    tol = bf16_ulp(torch.maximum(a.abs(), b.abs())) + b.abs().amax(dim=1, keepdim=True) * 2.0 ** -18
    bad = d > tol
    assert not bad.any(), f"{int(bad.sum())} saved FC1 values differ by more than one bf16 ulp"
    return None
