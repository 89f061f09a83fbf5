"""Pins the CPU oracle (oracle/moe_oracle.py) before it is trusted.

* routing: pure-Python brute-force stable sort on small inputs, a hand-made
  known answer, and the reference's invariants
  (tests/function/test_single_kernel_stable_scatter.py:17-67,121-179 of the
  reference: a permutation, non-decreasing expert ids, offsets = cumsum of
  counts, inverse with -1 for drops), including the full Kimi shape.
* combine: integer-valued rows make the fp32 slot sum exact
  (cf. tests/function/test_single_kernel_reduce.py:41-77 of the reference).
* forward / backward: an independent fp64 per-token evaluation and
  torch.autograd of it; a dropped term, wrong expert, transposed weight or
  sign error moves the result far beyond the bf16 tolerance used here.
"""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from tests._numeric import assert_rel


def brute_force_route(sel, E, k):
    flat = [int(v) for v in np.asarray(sel).reshape(-1)]
    pairs = [(e, r) for r, e in enumerate(flat) if 0 <= e < E]
    pairs.sort(key=lambda p: (p[0], p[1]))  # stable by expert == by (expert, route)
    send = [r for _, r in pairs]
    counts = [sum(1 for e, _ in pairs if e == x) for x in range(E)]
    r2s = [-1] * len(flat)
    for i, r in enumerate(send):
        r2s[r] = i
    return send, counts, r2s


def test_route_known_answer():
    sel = np.array([[2, 0], [0, 5], [1, 2], [-1, 2]], dtype=np.int32)  # 5 is out of range for E=3
    tb = O.route(sel, 3, 2)
    assert tb["send_route"].tolist() == [0 + 1, 2, 4, 0, 5, 7]
    assert tb["send_token"].tolist() == [0, 1, 2, 0, 2, 3]
    assert tb["counts"].tolist() == [2, 1, 3]
    assert tb["offsets"].tolist() == [0, 2, 3, 6]
    assert tb["route_to_send"].tolist() == [3, 0, 1, -1, 2, 4, -1, 5]


@pytest.mark.parametrize("seed", range(6))
def test_route_brute_force(seed):
    rng = np.random.default_rng(seed)
    E = int(rng.integers(1, 40))
    k = int(rng.integers(1, 9))
    T = int(rng.integers(0, 60))
    sel = rng.integers(-2, E + 3, size=(T, k)).astype(np.int32)
    tb = O.route(sel, E, k)
    send, counts, r2s = brute_force_route(sel, E, k)
    assert tb["send_route"].tolist() == send
    assert tb["counts"].tolist() == counts
    assert tb["route_to_send"].tolist() == r2s
    assert tb["send_token"].tolist() == [r // k for r in send]


@pytest.mark.parametrize("E,k,T", [(896, 16, 4096), (32, 8, 16384), (1, 4, 100)])
def test_route_invariants_large(E, k, T):
    rng = np.random.default_rng(E)
    sel = rng.integers(0, E, size=(T, k)).astype(np.int32)
    sel[0, 0] = -1
    sel[1, 1 % k] = E
    tb = O.route(sel, E, k)
    flat = sel.reshape(-1)
    send = tb["send_route"]
    experts = flat[send]
    assert np.all(np.diff(experts) >= 0)
    for e in range(E):  # within an expert, route ids ascend (stability)
        a, b = tb["offsets"][e], tb["offsets"][e + 1]
        assert np.all(np.diff(send[a:b]) > 0)
    assert np.array_equal(np.cumsum(tb["counts"]), tb["offsets"][1:])
    valid = (flat >= 0) & (flat < E)
    assert sorted(send.tolist()) == np.nonzero(valid)[0].tolist()
    assert np.all(tb["route_to_send"][~valid] == -1)
    assert np.array_equal(tb["route_to_send"][send], np.arange(send.size))


def _small_case(seed=0, T=24, H=32, inter=16, E=5, k=3, drop=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    sel = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
    if drop:
        sel[0, 0] = -1
        sel[3, 1] = E
    rw = torch.softmax(torch.randn(T, k, generator=g), dim=-1)
    w1 = (torch.randn(E, H, 2 * inter, generator=g) * 0.2).to(torch.bfloat16)
    w2 = (torch.randn(E, inter, H, generator=g) * 0.2).to(torch.bfloat16).transpose(1, 2)
    dy = torch.randn(T, H, generator=g).to(torch.bfloat16)
    return x, sel, w1, w2, rw, dy


def test_combine_integer_exact():
    # rows with small integers: the fp32 slot sum and the bf16 store are exact
    T, k, H = 7, 3, 16
    sel = torch.tensor([[0, 1, 2]] * T, dtype=torch.int32)
    sel[2, 1] = -1
    tb = O.route(sel.numpy(), 3, k)
    y = torch.arange(T * k * H, dtype=torch.float32).reshape(T * k, H) % 17
    r2s = torch.from_numpy(tb["route_to_send"]).long().view(T, k)
    out = torch.zeros(T, H)
    for j in range(k):
        m = r2s[:, j] >= 0
        out[m] += y[r2s[m, j]]
    expect = torch.zeros(T, H)
    send = tb["send_route"]
    for i, r in enumerate(send):
        expect[r // k] += y[i]
    assert torch.equal(out, expect)


@pytest.mark.parametrize("activation", ["swiglu", "clamp_swiglu", "situglu"])
def test_forward_matches_fp64_dense(activation):
    x, sel, w1, w2, rw, _ = _small_case(seed=1)
    kw = dict(activation=activation, situ_beta=1.5, situ_linear_beta=2.0 if activation == "situglu" else None,
              clamp_limit=0.3)
    out, _ = O.forward(x, sel, w1, w2, rw, **kw)
    ref = O.reference_autograd(x, sel, w1, w2, rw, torch.zeros(x.shape), **kw)
    assert_rel(out, ref["out"], 2e-2, "forward")
    sub = O.forward_tokens(x, sel, w1, w2, rw, [0, 3, 7], **kw)
    assert torch.equal(sub, out[[0, 3, 7]])


@pytest.mark.parametrize("activation", ["swiglu", "clamp_swiglu", "situglu"])
def test_backward_matches_autograd(activation):
    x, sel, w1, w2, rw, dy = _small_case(seed=2)
    kw = dict(activation=activation, situ_beta=1.5, situ_linear_beta=2.0 if activation == "situglu" else None,
              clamp_limit=0.3)
    _, st = O.forward(x, sel, w1, w2, rw, **kw)
    g = O.backward(st, dy)
    ref = O.reference_autograd(x, sel, w1, w2, rw, dy, **kw)
    assert_rel(g["grad_hidden"], ref["grad_hidden"], 2e-2, "grad_hidden")
    assert_rel(g["grad_routing_weights"], ref["grad_routing_weights"], 3e-2, "grad_rw")
    assert_rel(g["grad_gate_up"], ref["grad_gate_up"], 2e-2, "grad_gate_up")
    assert_rel(g["grad_fc2"], ref["grad_fc2"], 2e-2, "grad_fc2")
    # dropped routes get zero routing-weight gradient
    assert g["grad_routing_weights"][0, 0] == 0 and g["grad_routing_weights"][3, 1] == 0
