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


# --------------------------------------------------------------------- saved FC1 formats
def test_e4m3fn_codes_round_trip_through_the_quantizer_cast():
    """Every finite E4M3 code: its closed-form value converts back to the same
    code, and the cast's decode equals the closed form."""
    for code in range(256):
        v = O.e4m3fn_value(code)
        if v != v:  # NaN codes 0x7F / 0xFF
            assert code & 0x7F == 0x7F
            continue
        t = torch.tensor([v], dtype=torch.float32).to(torch.float8_e4m3fn)
        if v == 0.0:
            assert t.view(torch.uint8).item() in (0x00, 0x80)
        else:
            assert t.view(torch.uint8).item() == code, hex(code)
        assert torch.tensor([code], dtype=torch.uint8).view(torch.float8_e4m3fn).float().item() == v


def test_e4m3fn_ties_to_even_and_saturation():
    pos = [O.e4m3fn_value(c) for c in range(0x7F)]  # 0 .. 448, increasing
    assert pos == sorted(pos) and pos[-1] == 448.0
    for c in range(0x7E):
        lo, hi = pos[c], pos[c + 1]
        mid = (lo + hi) / 2
        even = c if c % 2 == 0 else c + 1
        got = torch.tensor([mid, mid - (hi - lo) / 8, mid + (hi - lo) / 8]).to(torch.float8_e4m3fn).view(torch.uint8)
        assert got.tolist() == [even, c, c + 1], (c, lo, hi)
    # the quantizer saturates: clamp then cast
    q, s = O.quantize_fc1(torch.full((1, 256), 3.0), "fp8")
    assert torch.all(q.float() == 448.0) and torch.allclose(s, torch.full((1, 2), 3.0 / 448.0))


def test_quantize_fc1_fp8_group_invariants():
    g = torch.Generator().manual_seed(3)
    I = 256
    gu = O.bf16(torch.randn(40, 2 * I, generator=g) * torch.logspace(-3, 2, 40)[:, None])
    gu[7] = 0.0                       # an all-zero row: q = 0, scale = 1/448
    gu[9, :128] = 0.0                 # one zero group
    q, s = O.quantize_fc1(gu, "fp8")
    assert q.dtype == torch.float8_e4m3fn and q.shape == gu.shape and s.shape == (40, 2 * I // 128)
    qg = q.float().view(40, -1, 128)
    amax = gu.view(40, -1, 128).abs().amax(2)
    nz = amax > 0
    assert torch.all(qg.abs().amax(2)[nz] == 448.0)
    assert torch.all(qg[~nz] == 0) and torch.all(s[~nz] == 1.0 / 448.0)
    assert torch.allclose(s[nz], amax[nz] / 448.0, rtol=1e-7, atol=0)
    # gate groups first, then up groups
    assert torch.equal(s[:, 0], torch.where(gu[:, :128].abs().amax(1) > 0, gu[:, :128].abs().amax(1), torch.ones(40)) / 448.0)
    d = O.dequantize_fc1(q, s)
    err = (d - gu).abs().view(40, -1, 128)
    bound = gu.view(40, -1, 128).abs() * 2.0 ** -4 + (amax / 448.0 * 2.0 ** -10)[..., None] * 1.001
    assert torch.all(err <= bound)


def test_quantize_fc1_fp16_is_exact_for_bf16_values():
    g = torch.Generator().manual_seed(4)
    gu = O.bf16(torch.randn(16, 256, generator=g) * 50)
    q, s = O.quantize_fc1(gu, "fp16")
    assert s is None and q.dtype == torch.float16 and torch.equal(q.float(), gu)


@pytest.mark.parametrize("fmt", ["fp16", "fp8"])
def test_backward_with_narrow_fc1_save_stays_close(fmt):
    """The backward reads the saved FC1 through the narrow format only: fp16
    keeps the bf16 values exactly, fp8 moves the gradients by at most a few
    percent of their scale."""
    T, H, I, E, k = 48, 64, 128, 4, 2
    g = torch.Generator().manual_seed(8)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    sel = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
    w1 = (torch.randn(E, H, 2 * I, generator=g) * 0.1).to(torch.bfloat16)
    w2 = (torch.randn(E, H, I, generator=g) * 0.1).to(torch.bfloat16)
    rw = torch.softmax(torch.randn(T, k, generator=g), 1)
    dy = torch.randn(T, H, generator=g).to(torch.bfloat16)
    _, st_b = O.forward(x, sel, w1, w2, rw)
    _, st_n = O.forward(x, sel, w1, w2, rw, save_fc1_dtype=fmt)
    rb, rn = O.backward(st_b, dy), O.backward(st_n, dy)
    for key in ("grad_hidden", "grad_gate_up", "grad_routing_weights"):
        a, b = rn[key].float(), rb[key].float()
        rel = float((a - b).abs().max() / b.abs().max())
        if fmt == "fp16":
            assert rel == 0.0, key
        else:
            assert rel < 0.1, (key, rel)
    assert torch.equal(rn["grad_fc2"], rb["grad_fc2"])  # dW2 does not read the FC1 save


def test_quantize_fc1_multiplier_is_correctly_rounded():
    """448 / amax is one correctly rounded fp32 division (as the device epilogue
    computes it): for amax = 6, 0.28125 * fp32(448 / 6) is exactly 21, a tie
    between the E4M3 codes for 20 and 22 that rounds to the even one (20)."""
    gu = torch.zeros(1, 256)
    gu[0, 0], gu[0, 1] = 6.0, 0.28125
    q, s = O.quantize_fc1(gu, "fp8")
    assert q.view(torch.uint8)[0, 1].item() == 0x5A and q.float()[0, 1].item() == 20.0
    assert q.float()[0, 0].item() == 448.0 and s[0, 0].item() == torch.tensor(6.0 / 448.0).item()


def test_backward_recompute_act_matches_saved_for_bf16():
    """With the bf16 save, the recomputed activation equals the saved one, so
    recompute mode leaves every gradient unchanged."""
    T, H, I, E, k = 40, 64, 128, 4, 2
    g = torch.Generator().manual_seed(12)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    sel = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
    w1 = (torch.randn(E, H, 2 * I, generator=g) * 0.1).to(torch.bfloat16)
    w2 = (torch.randn(E, H, I, generator=g) * 0.1).to(torch.bfloat16)
    rw = torch.softmax(torch.randn(T, k, generator=g), 1)
    dy = torch.randn(T, H, generator=g).to(torch.bfloat16)
    _, st = O.forward(x, sel, w1, w2, rw)
    a, b = O.backward(st, dy), O.backward(st, dy, recompute_act=True)
    for key in ("grad_hidden", "grad_fc2", "grad_gate_up", "grad_routing_weights"):
        assert torch.equal(a[key], b[key])


# --------------------------------------------------------------------- sampled backward helpers
@pytest.mark.parametrize("activation", ["swiglu", "clamp_swiglu", "situglu"])
def test_backward_tokens_equals_full_backward(activation):
    """backward_tokens over every token evaluates each expert's complete row
    set with the same GEMM shapes as forward/backward: bit-identical output,
    grad_hidden and grad_routing_weights. A subset agrees to bf16 rounding
    (the only difference is the GEMM's row count)."""
    x, sel, w1, w2, rw, dy = _small_case(seed=5, T=40, E=6, k=3)
    kw = dict(activation=activation, situ_beta=1.5, situ_linear_beta=2.0 if activation == "situglu" else None,
              clamp_limit=0.3)
    out, st = O.forward(x, sel, w1, w2, rw, **kw)
    g = O.backward(st, dy)
    full = O.backward_tokens(x, sel, w1, w2, rw, dy, range(x.shape[0]), **kw)
    assert torch.equal(full["out"], out)
    assert torch.equal(full["grad_hidden"], g["grad_hidden"])
    assert torch.equal(full["grad_routing_weights"], g["grad_routing_weights"])
    toks = [0, 3, 17, 39]
    sub = O.backward_tokens(x, sel, w1, w2, rw, dy, toks, **kw)
    for name, ref in (("out", out), ("grad_hidden", g["grad_hidden"])):
        d = (sub[name].float() - ref[toks].float()).abs()
        assert float(d.max()) <= 2 ** -7 * float(ref[toks].float().abs().max()), name
    d = (sub["grad_routing_weights"] - g["grad_routing_weights"][toks]).abs()
    assert float(d.max()) <= 2 ** -7 * float(g["grad_routing_weights"].abs().max())
    assert sub["grad_routing_weights"][0, 0] == 0          # dropped route


@pytest.mark.parametrize("fmt", ["fp16", "fp8"])
def test_sampled_backward_reads_the_narrow_save(fmt):
    """With a narrowed FC1 save, backward_tokens / backward_expert over the
    complete row sets equal the full backward reading the same save."""
    x, sel, w1, w2, rw, dy = _small_case(seed=8, T=32, H=32, inter=128, E=4, k=2)
    _, st = O.forward(x, sel, w1, w2, rw, save_fc1_dtype=fmt)
    g = O.backward(st, dy)
    full = O.backward_tokens(x, sel, w1, w2, rw, dy, range(x.shape[0]), save_fc1_dtype=fmt)
    assert torch.equal(full["grad_hidden"], g["grad_hidden"])
    assert torch.equal(full["grad_routing_weights"], g["grad_routing_weights"])
    for e in range(4):
        dgu, dfc2 = O.backward_expert(x, sel, w1, w2, rw, dy, e, save_fc1_dtype=fmt)
        assert torch.equal(dgu, g["grad_gate_up"][e]) and torch.equal(dfc2, g["grad_fc2"][e])
    # and the narrow save changes the gradients (the format is really applied)
    if fmt == "fp8":
        ref16 = O.backward_tokens(x, sel, w1, w2, rw, dy, range(x.shape[0]))
        assert not torch.equal(ref16["grad_hidden"], full["grad_hidden"])


@pytest.mark.parametrize("activation", ["swiglu", "clamp_swiglu"])
def test_backward_expert_equals_full_backward(activation):
    """backward_expert(e) is the e-th slice of the full weight gradients, bit
    for bit, for every expert (including one with no rows)."""
    x, sel, w1, w2, rw, dy = _small_case(seed=6, T=30, E=7, k=2)
    sel[sel == 4] = 6                                        # expert 4 gets no rows
    kw = dict(activation=activation, clamp_limit=0.3)
    _, st = O.forward(x, sel, w1, w2, rw, **kw)
    g = O.backward(st, dy)
    for e in range(7):
        dgu, dfc2 = O.backward_expert(x, sel, w1, w2, rw, dy, e, **kw)
        assert torch.equal(dgu, g["grad_gate_up"][e]), e
        assert torch.equal(dfc2, g["grad_fc2"][e]), e
    assert torch.count_nonzero(g["grad_gate_up"][4]) == 0
