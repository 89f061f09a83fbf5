"""CPU checks of the saved-FC1 comparison helpers the GPU tests rely on."""

import math

import torch

from oracle import moe_oracle as O
from tests._fc1_save import bf16_ulp, e4m3_magnitude_index


def test_e4m3_index_orders_every_finite_code():
    """Sorting the 252 finite non-zero E4M3 codes by their closed-form value
    gives consecutive magnitude indices: one index step is one
    representable-value step."""
    codes = [c for c in range(256) if not math.isnan(O.e4m3fn_value(c)) and c & 0x7F]
    vals = [O.e4m3fn_value(c) for c in codes]
    q = torch.tensor(codes, dtype=torch.uint8).view(torch.float8_e4m3fn)
    idx = e4m3_magnitude_index(q).tolist()
    by_value = [i for _, i in sorted(zip(vals, idx))]
    assert by_value == sorted(idx)
    pos = sorted(i for i in idx if i > 0)
    assert pos == list(range(1, 127))


def test_bf16_ulp_is_the_spacing():
    x = torch.tensor([1.0, 1.5, 3.0, -0.05, 448.0, 1e-3]).to(torch.bfloat16).float()
    u = bf16_ulp(x)
    nxt = (x.abs().to(torch.bfloat16).view(torch.int16) + 1).view(torch.bfloat16).float()
    assert torch.equal(nxt - x.abs(), u)
