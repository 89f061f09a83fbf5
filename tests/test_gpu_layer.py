"""Layer-level parity: FusedMoEForward / moe_backward_triton / MegaMoEFunction
against the CPU oracle (GPU)."""

import math

import pytest
import torch

import mega_moe
from mega_moe.bench_configs import CASES, CaseSpec, make_inputs
from oracle import moe_oracle as O
from tests._numeric import GRAD_ATOL, GRAD_RTOL, OUTPUT_ATOL, OUTPUT_RTOL, assert_rel, cmp_grad

pytestmark = pytest.mark.gpu

SMALL = [
    CaseSpec("small_topk", 256, 256, 128, 8, 4, "softmax_topk", True),
    CaseSpec("small_skew", 384, 256, 256, 16, 4, "zipf", True),
    CaseSpec("toy_bf16", 512, 256, 512, 8, 2, "softmax_topk", True),
]


def _op(spec, activation="swiglu", **cfg):
    config = mega_moe.MoEForwardConfig(activation=activation, **cfg)
    return mega_moe.FusedMoEForward(None, max_tokens_per_rank=spec.tokens, hidden_size=spec.hidden,
                                    top_k=spec.top_k, num_experts=spec.experts, config=config)


def _act_kw(activation):
    return dict(activation=activation, situ_beta=1.0 if activation != "situglu" else 2.0,
                situ_linear_beta=3.0 if activation == "situglu" else None,
                clamp_limit=7.0 if activation != "clamp_swiglu" else 0.05)


@pytest.mark.parametrize("spec", SMALL, ids=lambda s: s.name)
@pytest.mark.parametrize("activation", ["swiglu", "clamp_swiglu", "situglu"])
def test_forward_backward_parity(spec, activation):
    inp = make_inputs(spec, device="cuda", seed=7, weight_scale=0.1)
    sel = inp["selected"].clone()
    sel[0, 0] = -1                      # dropped routes (reference drop_frac cases)
    sel[5, 1] = spec.experts
    kw = _act_kw(activation)
    cfg = {k: v for k, v in kw.items() if k != "activation"}
    op = _op(spec, activation, **cfg)
    out, saved = op.forward(inp["x"], sel, inp["gate_up"], inp["down"], inp["rw"], return_saved=True)
    saved["_keep_grad_recv_hidden_sorted"] = True
    g = mega_moe.moe_backward_triton(saved, inp["dy"], peer_mem=None)
    torch.cuda.synchronize()
    ref_out, st = O.forward(inp["x"].cpu(), sel.cpu(), inp["gate_up"].cpu(), inp["down"].cpu(),
                            inp["rw"].cpu(), **kw)
    ref = O.backward(st, inp["dy"].cpu())
    assert_rel(out, ref_out, 2e-2, "output")
    torch.testing.assert_close(out.float().cpu(), ref_out.float(), rtol=OUTPUT_RTOL, atol=OUTPUT_ATOL)
    for name in ("grad_hidden", "grad_routing_weights", "grad_fc2", "grad_gate_up"):
        assert_rel(g[name], ref[name], 2e-2, name)
        assert cmp_grad(g[name], ref[name], GRAD_RTOL, GRAD_ATOL) == 0, name
    assert g["grad_routing_weights"][0, 0] == 0 and g["grad_routing_weights"][5, 1] == 0
    # expert-major intermediates (reference tests/_moe_baselines.py:208-225)
    m = int(saved["split_size_cum_per_expert"][-1])
    assert "grad_fc2_out_sorted" in g and g["grad_fc2_out_sorted"].shape == (m, spec.hidden)
    assert torch.equal(g["grad_fc2_out_sorted"].float().cpu(), ref["grad_fc2_out_sorted"])
    assert_rel(g["grad_recv_hidden_sorted"], ref["grad_recv_hidden_sorted"], 2e-2, "grad_recv_hidden_sorted")
    assert_rel(g["grad_swiglu"][:m], ref["grad_swiglu"], 2e-2, "grad_swiglu")
    assert_rel(g["grad_fc1_output"][:m], ref["grad_fc1_output"], 2e-2, "grad_fc1_output")
    # unpacked views follow the reference's [E, F, H] layout
    I = spec.inter
    assert torch.equal(g["grad_fc1_1"], g["grad_gate_up"][:, :, :I].transpose(1, 2))


def test_routing_plan_and_dispatch_fc1():
    spec = SMALL[0]
    inp = make_inputs(spec, device="cuda", seed=3)
    op = _op(spec)
    sel = inp["selected"]
    plan = op.build_routing_plan(sel)
    ref = O.route(sel.cpu().numpy(), spec.experts, spec.top_k)
    assert plan.num_received_routes == int(ref["offsets"][-1])
    assert plan.send_route_indices.cpu().numpy().tolist() == ref["send_route"].tolist()
    assert plan.stable_sort_indices.cpu().numpy().tolist() == ref["stable_sort_indices"].tolist()
    assert plan.received_expert_offsets.cpu().numpy().tolist() == ref["offsets"].tolist()
    res = op.dispatch_fc1(inp["x"], sel, plan, inp["gate_up"], routing_weights=inp["rw"])
    torch.cuda.synchronize()
    st = torch.from_numpy(ref["send_token"]).long()
    assert torch.equal(res.dispatched_tokens.cpu(), inp["x"].cpu()[st])
    xp = inp["x"].float().cpu()[st]
    w1 = inp["gate_up"].float().cpu()
    o = ref["offsets"]
    gu = torch.cat([xp[o[e]:o[e + 1]] @ w1[e] for e in range(spec.experts)])
    assert_rel(res.fc1_output, gu, 1e-2, "fc1_output")


@pytest.mark.parametrize("fmt", ["bf16", "fp8"])
def test_autograd_function_matches_backward(fmt):
    spec = SMALL[0]
    inp = make_inputs(spec, device="cuda", seed=11, weight_scale=0.1)
    op = _op(spec, save_fc1_dtype=fmt)
    x = inp["x"].clone().requires_grad_(True)
    rw = inp["rw"].clone().requires_grad_(True)
    w1 = inp["gate_up"].clone().requires_grad_(True)
    w2 = inp["down"].contiguous().clone().requires_grad_(True)
    out = mega_moe.MegaMoEFunction.apply(op, x, rw, inp["selected"], w1, w2, torch.empty(1, device="cuda"), None)
    out.backward(inp["dy"])
    torch.cuda.synchronize()
    ref_out, st = O.forward(inp["x"].cpu(), inp["selected"].cpu(), inp["gate_up"].cpu(), w2.detach().cpu(),
                            inp["rw"].cpu(), save_fc1_dtype=fmt)
    ref = O.backward(st, inp["dy"].cpu())
    assert_rel(out.detach(), ref_out, 2e-2, "out")
    assert_rel(x.grad, ref["grad_hidden"], 2e-2, "dx")
    assert_rel(rw.grad, ref["grad_routing_weights"], 2e-2, "drw")
    assert_rel(w1.grad, ref["grad_gate_up"], 2e-2, "dw1")
    assert_rel(w2.grad, ref["grad_fc2"], 2e-2, "dw2")
    # a second forward supersedes the first plan: its backward must be rejected
    out2 = mega_moe.MegaMoEFunction.apply(op, x, rw, inp["selected"], w1, w2, torch.empty(1, device="cuda"), None)
    out3 = mega_moe.MegaMoEFunction.apply(op, x, rw, inp["selected"], w1, w2, torch.empty(1, device="cuda"), None)
    with pytest.raises(RuntimeError, match="superseded"):
        out2.sum().backward()
    del out3


def test_single_kernel_snapshot_shared_operator():
    """enable_single_kernel_forward: one operator shared by two same-shape
    layers runs forward A, forward B, backward B, backward A (the reference's
    snapshot gate, ops/function.py:143-158 with _single_saved_adapter.py:369);
    the default mode keeps rejecting the superseded backward."""
    spec = SMALL[0]
    op = _op(spec, enable_single_kernel_forward=True)
    layers = []
    for seed in (21, 22):
        inp = make_inputs(spec, device="cuda", seed=seed, weight_scale=0.1)
        x = inp["x"].clone().requires_grad_(True)
        rw = inp["rw"].clone().requires_grad_(True)
        w1 = inp["gate_up"].clone().requires_grad_(True)
        w2 = inp["down"].contiguous().clone().requires_grad_(True)
        out = mega_moe.MegaMoEFunction.apply(op, x, rw, inp["selected"], w1, w2, torch.empty(1, device="cuda"),
                                             None)
        layers.append((inp, x, rw, w1, w2, out))
    for inp, x, rw, w1, w2, out in reversed(layers):
        out.backward(inp["dy"])
    torch.cuda.synchronize()
    for inp, x, rw, w1, w2, out in layers:
        ref_out, st = O.forward(inp["x"].cpu(), inp["selected"].cpu(), inp["gate_up"].cpu(),
                                w2.detach().cpu(), inp["rw"].cpu())
        ref = O.backward(st, inp["dy"].cpu())
        assert_rel(out.detach(), ref_out, 2e-2, "out")
        assert_rel(x.grad, ref["grad_hidden"], 2e-2, "dx")
        assert_rel(rw.grad, ref["grad_routing_weights"], 2e-2, "drw")
        assert_rel(w1.grad, ref["grad_gate_up"], 2e-2, "dw1")
        assert_rel(w2.grad, ref["grad_fc2"], 2e-2, "dw2")


def _sample_tokens(ref, spec, experts, n):
    """Tokens whose rows sit where tiling goes wrong first: the first and last
    rows of the given experts (hottest: longest run of full tiles; ragged:
    a short last tile), the first and last token, then evenly spaced tokens
    up to ``n``."""
    off, st = ref["offsets"], ref["send_token"]
    picks = [0, spec.tokens - 1]
    for e in experts:
        a, b = int(off[e]), int(off[e + 1])
        picks += [int(t) for t in st[a:min(b, a + 4)]] + [int(t) for t in st[max(a, b - 8):b]]
    step = max(1, spec.tokens // n)
    t = 1
    while len(dict.fromkeys(picks)) < n:
        picks.append(t)
        t = (t + step) % spec.tokens
    return list(dict.fromkeys(picks))[:n]


def _probe_experts(counts):
    """(hottest, median, ragged): the ragged one has the shortest non-empty
    remainder past a multiple of 128 rows (a last tile holding a few rows)."""
    order = sorted(range(len(counts)), key=lambda e: (int(counts[e]), e))
    hottest, median = order[-1], order[len(order) // 2]
    rag = [e for e in order if counts[e] % 128 and e not in (hottest, median)]
    ragged = min(rag, key=lambda e: (int(counts[e]) % 128, -int(counts[e]))) if rag else order[0]
    return hottest, median, ragged


@pytest.mark.parametrize("name,fmt,activation", [
    ("e32", "bf16", "swiglu"), ("qwen", "bf16", "swiglu"), ("skew", "bf16", "swiglu"), ("kimi", "bf16", "swiglu"),
    ("kimi", "fp8", "swiglu"), ("kimi8k", "bf16", "swiglu"), ("qwen", "bf16", "situglu"),
    ("qwen", "fp16", "clamp_swiglu"), ("qwen", "fp8", "swiglu"), ("dsv3", "bf16", "swiglu")])
def test_full_size_sampled_parity(name, fmt, activation):
    """BASELINE sizes and seeds, forward + backward: routing bit-exact; output
    rows, grad_hidden rows and grad_routing_weights rows of 64 sampled
    tokens (hottest expert, a ragged last tile, spread tokens); the full
    weight gradients of three experts (hottest, median, ragged) -- all
    against the CPU oracle, max relative error <= 2e-2 plus the reference's
    GRAD element check. (E32 is a forward-only config; its backward is
    checked too.) The Kimi layer also runs with the FP8 FC1 save, the
    backward reading the E4M3 values and scales (128-row tiles), the
    Qwen-like layer with the SiTU-GLU and clamped SwiGLU activations and the
    FP8 save (256-row register-staged tiles), and the DeepSeek-V3-like layer
    (256 experts averaging 128 rows, 256-row tiles)."""
    spec = CASES[name]
    inp = make_inputs(spec, device="cuda", seed=1234)
    kw = _act_kw(activation)
    op = _op(spec, activation, save_fc1_dtype=fmt, **{k: v for k, v in kw.items() if k != "activation"})
    x, sel, w1, w2, rw, dy = inp["x"], inp["selected"], inp["gate_up"], inp["down"], inp["rw"], inp["dy"]
    out, saved = op.forward(x, sel, w1, w2, rw, return_saved=True)
    g = mega_moe.moe_backward_triton(saved, dy)
    torch.cuda.synchronize()
    ref = O.route(sel.cpu().numpy(), spec.experts, spec.top_k)
    nv = int(ref["offsets"][-1])
    assert saved["split_size_cum_per_expert"].cpu().numpy().tolist() == ref["offsets"].tolist()
    assert saved["send_route_indices"][:nv].cpu().numpy().tolist() == ref["send_route"].tolist()
    assert saved["send_token_indices"][:nv].cpu().numpy().tolist() == ref["send_token"].tolist()
    assert saved["route_to_send"].cpu().numpy().tolist() == ref["route_to_send"].tolist()
    experts = _probe_experts(ref["counts"])
    print(f"[{name}] probe experts (hottest, median, ragged) = {experts}, rows = "
          f"{[int(ref['counts'][e]) for e in experts]}", flush=True)
    toks = _sample_tokens(ref, spec, (experts[0], experts[2]), 64)
    sub = O.backward_tokens(x, sel, w1, w2, rw, dy, toks, save_fc1_dtype=fmt, **kw)
    assert_rel(out[toks], sub["out"], 2e-2, f"{name} output rows")
    for key in ("grad_hidden", "grad_routing_weights"):
        assert_rel(g[key][toks], sub[key], 2e-2, f"{name} {key} rows")
        assert cmp_grad(g[key][toks], sub[key], GRAD_RTOL, GRAD_ATOL) == 0, key
    for e in experts:
        dgu, dfc2 = O.backward_expert(x, sel, w1, w2, rw, dy, e, save_fc1_dtype=fmt, **kw)
        assert_rel(g["grad_gate_up"][e], dgu, 2e-2, f"{name} grad_gate_up[{e}]")
        assert_rel(g["grad_fc2"][e], dfc2, 2e-2, f"{name} grad_fc2[{e}]")
        assert cmp_grad(g["grad_gate_up"][e], dgu, GRAD_RTOL, GRAD_ATOL) == 0
        assert cmp_grad(g["grad_fc2"][e], dfc2, GRAD_RTOL, GRAD_ATOL) == 0
    del inp, out, saved, g, x, sel, w1, w2, rw, dy
    torch.cuda.empty_cache()


def test_kimi_layer_at_16k_tokens():
    """The Kimi-scale layer at 16384 tokens (the reference's largest bench
    size per rank): 262144 routes, so every row offset and output index
    passes 2^28 elements; forward + backward on sampled tokens and one
    expert's weight gradients against the oracle."""
    base = CASES["kimi"]
    spec = CaseSpec("kimi16k", 16384, base.hidden, base.inter, base.experts, base.top_k, base.routing, True)
    inp = make_inputs(spec, device="cuda", seed=77)
    op = _op(spec)
    x, sel, w1, w2, rw, dy = inp["x"], inp["selected"], inp["gate_up"], inp["down"], inp["rw"], inp["dy"]
    out, saved = op.forward(x, sel, w1, w2, rw, return_saved=True)
    g = mega_moe.moe_backward_triton(saved, dy)
    torch.cuda.synchronize()
    ref = O.route(sel.cpu().numpy(), spec.experts, spec.top_k)
    assert saved["route_to_send"].cpu().numpy().tolist() == ref["route_to_send"].tolist()
    toks = [0, 1, 8191, 8192, 16382, 16383]
    sub = O.backward_tokens(x, sel, w1, w2, rw, dy, toks)
    assert_rel(out[toks], sub["out"], 2e-2, "16k output rows")
    assert_rel(g["grad_hidden"][toks], sub["grad_hidden"], 2e-2, "16k grad_hidden rows")
    assert_rel(g["grad_routing_weights"][toks], sub["grad_routing_weights"], 2e-2, "16k grad_rw rows")
    e = int(sel[16383, 0])                      # an expert whose rows reach the end of the route space
    dgu, dfc2 = O.backward_expert(x, sel, w1, w2, rw, dy, e)
    assert_rel(g["grad_gate_up"][e], dgu, 2e-2, "16k grad_gate_up")
    assert_rel(g["grad_fc2"][e], dfc2, 2e-2, "16k grad_fc2")
    del inp, out, saved, g, x, sel, w1, w2, rw, dy
    torch.cuda.empty_cache()


def test_deterministic_and_finalize_reuse():
    """No atomics anywhere: two runs of forward + backward are bit-identical
    (including a Zipf-skewed routing with ragged tiles); after finalize()
    releases the workspaces, the next forward re-reserves them and matches."""
    spec = CaseSpec("det", 1024, 512, 256, 24, 6, "zipf", True)
    inp = make_inputs(spec, device="cuda", seed=19, weight_scale=0.1)
    op = _op(spec)
    args = (inp["x"], inp["selected"], inp["gate_up"], inp["down"], inp["rw"])
    names = ("grad_hidden", "grad_routing_weights", "grad_fc2", "grad_gate_up")

    def run():
        out, saved = op.forward(*args, return_saved=True)
        g = mega_moe.moe_backward_triton(saved, inp["dy"])
        return [out.clone()] + [g[n].clone() for n in names]

    a, b = run(), run()
    for n, x, y in zip(("out",) + names, a, b):
        assert torch.equal(x, y), n
    op.finalize()
    assert op._workspaces.nbytes() == 0
    c = run()
    for n, x, y in zip(("out",) + names, a, c):
        assert torch.equal(x, y), f"after finalize: {n}"


def test_validation_errors_on_device():
    spec = SMALL[0]
    inp = make_inputs(spec, device="cuda", seed=1)
    op = _op(spec)
    x, sel, w1, w2, rw = inp["x"], inp["selected"], inp["gate_up"], inp["down"], inp["rw"]
    with pytest.raises(ValueError, match="max_tokens_per_rank"):
        op.forward(torch.cat([x, x]), torch.cat([sel, sel]), w1, w2, torch.cat([rw, rw]))
    with pytest.raises(TypeError):
        op.forward(x.float(), sel, w1, w2, rw)
    with pytest.raises(ValueError):
        op.forward(x, sel, w1, w2, rw.to(torch.bfloat16))
    with pytest.raises(ValueError):
        op.forward(x, sel, w1[:, :, :-2].contiguous(), w2, rw)
    with pytest.raises(ValueError):
        op.forward(x[:, :128].contiguous(), sel, w1, w2, rw)
    with pytest.raises(ValueError, match="contiguous"):
        op.forward(x, sel, w1.transpose(1, 2), w2, rw)
    # single-stream rule (reference forward.py:1929-1936)
    op.forward(x, sel, w1, w2, rw)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with pytest.raises(RuntimeError, match="single-stream"):
            op.forward(x, sel, w1, w2, rw)
    torch.cuda.synchronize()


def test_empty_batch():
    spec = SMALL[0]
    inp = make_inputs(spec, device="cuda", seed=1)
    op = _op(spec)
    x0 = inp["x"][:0]
    out = op.forward(x0, inp["selected"][:0], inp["gate_up"], inp["down"], inp["rw"][:0])
    assert out.shape == (0, spec.hidden)
    # backward of an empty batch: empty input gradients, zero weight gradients
    out, saved = op.forward(x0, inp["selected"][:0], inp["gate_up"], inp["down"], inp["rw"][:0],
                            return_saved=True)
    g = mega_moe.moe_backward_triton(saved, inp["dy"][:0])
    assert g["grad_hidden"].shape == (0, spec.hidden) and g["grad_routing_weights"].shape == (0, spec.top_k)
    assert g["grad_gate_up"].shape == inp["gate_up"].shape and torch.count_nonzero(g["grad_gate_up"]) == 0
    assert g["grad_fc2"].shape == inp["down"].shape and torch.count_nonzero(g["grad_fc2"]) == 0
    # and through the autograd function
    x = x0.clone().requires_grad_(True)
    rw = inp["rw"][:0].clone().requires_grad_(True)
    w1 = inp["gate_up"].clone().requires_grad_(True)
    w2 = inp["down"].contiguous().requires_grad_(True)
    y = mega_moe.MegaMoEFunction.apply(op, x, rw, inp["selected"][:0], w1, w2, torch.empty(1, device="cuda"), None)
    y.sum().backward()
    assert x.grad.shape == x0.shape and torch.count_nonzero(w1.grad) == 0 and torch.count_nonzero(w2.grad) == 0


def test_many_experts_layer():
    """E = 2048 (above the 4-wave scatter's 1024): forward + backward parity."""
    spec = CaseSpec("many_experts", 512, 256, 128, 2048, 4, "softmax_topk", True)
    inp = make_inputs(spec, device="cuda", seed=13, weight_scale=0.1)
    op = _op(spec)
    out, saved = op.forward(inp["x"], inp["selected"], inp["gate_up"], inp["down"], inp["rw"], return_saved=True)
    g = mega_moe.moe_backward_triton(saved, inp["dy"])
    torch.cuda.synchronize()
    ref_out, st = O.forward(inp["x"].cpu(), inp["selected"].cpu(), inp["gate_up"].cpu(), inp["down"].cpu(),
                            inp["rw"].cpu())
    ref = O.backward(st, inp["dy"].cpu())
    nv = int(st["tables"]["offsets"][-1])
    assert saved["send_route_indices"][:nv].cpu().numpy().tolist() == st["tables"]["send_route"].tolist()
    assert_rel(out, ref_out, 2e-2, "out")
    for name in ("grad_hidden", "grad_routing_weights", "grad_fc2", "grad_gate_up"):
        assert_rel(g[name], ref[name], 2e-2, name)


def test_all_routes_dropped_and_one_hot_expert():
    spec = SMALL[0]
    inp = make_inputs(spec, device="cuda", seed=4, weight_scale=0.1)
    op = _op(spec)
    dropped = torch.full_like(inp["selected"], spec.experts)
    out = op.forward(inp["x"], dropped, inp["gate_up"], inp["down"], inp["rw"])
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0
    hot = torch.zeros_like(inp["selected"])  # every route to expert 0 (reference all-to-rank-0 case)
    hot[:, 1:] = -1
    out, saved = op.forward(inp["x"], hot, inp["gate_up"], inp["down"], inp["rw"], return_saved=True)
    g = mega_moe.moe_backward_triton(saved, inp["dy"])
    torch.cuda.synchronize()
    ref_out, st = O.forward(inp["x"].cpu(), hot.cpu(), inp["gate_up"].cpu(), inp["down"].cpu(), inp["rw"].cpu())
    ref = O.backward(st, inp["dy"].cpu())
    assert_rel(out, ref_out, 2e-2, "out")
    for name in ("grad_hidden", "grad_routing_weights", "grad_fc2", "grad_gate_up"):
        assert_rel(g[name], ref[name], 2e-2, name)


@pytest.mark.parametrize("spec", SMALL, ids=lambda s: s.name)
@pytest.mark.parametrize("fmt", ["fp16", "fp8"])
def test_saved_fc1_formats(spec, fmt):
    """save_fc1_dtype fp16 / fp8 (reference config.py:178-186): the saved bytes
    equal the oracle's narrowing of this build's own bf16 save (bit exact,
    FP8 scales included), and the backward through the narrow save matches
    the oracle backward that reads the same format."""
    inp = make_inputs(spec, device="cuda", seed=21, weight_scale=0.1)
    sel = inp["selected"].clone()
    sel[3, 0] = -1
    args = (inp["x"], sel, inp["gate_up"], inp["down"], inp["rw"])
    _, sb = _op(spec).forward(*args, return_saved=True)
    out, sn = _op(spec, save_fc1_dtype=fmt).forward(*args, return_saved=True)
    g = mega_moe.moe_backward_triton(sn, inp["dy"])
    torch.cuda.synchronize()
    n = int(sb["split_size_cum_per_expert"][-1])
    ref_q, ref_s = O.quantize_fc1(sb["fc1_output"][:n].float().cpu(), fmt)
    got = sn["fc1_output"][:n].cpu()
    assert got.dtype == ref_q.dtype
    assert torch.equal(got.view(torch.uint8) if fmt == "fp8" else got, ref_q.view(torch.uint8) if fmt == "fp8" else ref_q)
    if fmt == "fp8":
        assert sn["fc1_scale_group_size"] == 128
        assert torch.equal(sn["fc1_output_scale"][:n].cpu(), ref_s)
    else:
        assert "fc1_output_scale" not in sn
    ref_out, st = O.forward(inp["x"].cpu(), sel.cpu(), inp["gate_up"].cpu(), inp["down"].cpu(), inp["rw"].cpu(),
                            save_fc1_dtype=fmt)
    ref = O.backward(st, inp["dy"].cpu())
    assert_rel(out, ref_out, 2e-2, "output")
    for name in ("grad_hidden", "grad_routing_weights", "grad_fc2", "grad_gate_up"):
        assert_rel(g[name], ref[name], 2e-2, name)


def test_fp8_save_needs_default_block():
    with pytest.raises(NotImplementedError):
        _op(SMALL[0], save_fc1_dtype="fp8", fc1_gemm_block_size_n=128)


@pytest.mark.parametrize("activation", ["swiglu", "clamp_swiglu", "situglu"])
def test_act_recompute_is_bit_exact_for_bf16_save(activation):
    """mm_gated_act over the saved bf16 FC1 output reproduces the forward's
    weighted activation bit for bit."""
    from mega_moe.ops import _kernels as K
    spec = SMALL[1]
    kw = _act_kw(activation)
    cfg = {k: v for k, v in kw.items() if k != "activation"}
    inp = make_inputs(spec, device="cuda", seed=31, weight_scale=0.1)
    _, sv = _op(spec, activation, **cfg).forward(inp["x"], inp["selected"], inp["gate_up"], inp["down"], inp["rw"],
                                                 return_saved=True)
    act = K.gated_act(sv["fc1_output"], sv["recv_weights_sorted"], sv["split_size_cum_per_expert"],
                      sv["total_routes"], **kw)
    torch.cuda.synchronize()
    n = int(sv["split_size_cum_per_expert"][-1])
    assert torch.equal(act[:n], sv["swiglu_out_weighted"][:n])


@pytest.mark.parametrize("fmt", ["bf16", "fp8"])
def test_saved_recompute_mode(fmt, monkeypatch):
    """MOE_SAVED_RECOMPUTE=1: the saved dict drops the weighted activation and
    the backward recomputes it from fc1_output (bf16: identical gradients;
    fp8: within tolerance of the oracle reading the same save)."""
    spec = SMALL[0]
    inp = make_inputs(spec, device="cuda", seed=33, weight_scale=0.1)
    args = (inp["x"], inp["selected"], inp["gate_up"], inp["down"], inp["rw"])
    _, s0 = _op(spec, save_fc1_dtype=fmt).forward(*args, return_saved=True)
    g0 = mega_moe.moe_backward_triton(s0, inp["dy"])
    monkeypatch.setenv("MOE_SAVED_RECOMPUTE", "1")
    _, s1 = _op(spec, save_fc1_dtype=fmt).forward(*args, return_saved=True)
    assert "swiglu_out_weighted" not in s1
    g1 = mega_moe.moe_backward_triton(s1, inp["dy"])
    torch.cuda.synchronize()
    names = ("grad_hidden", "grad_routing_weights", "grad_fc2", "grad_gate_up")
    if fmt == "bf16":
        for name in names:
            assert torch.equal(g1[name], g0[name]), name
    else:
        _, st = O.forward(*(t.cpu() for t in args), save_fc1_dtype=fmt)
        ref = O.backward(st, inp["dy"].cpu(), recompute_act=True)
        for name in names:
            assert_rel(g1[name], ref[name], 2e-2, name)


def test_backward_function_over_unpacked_weights():
    """MegaMoEBackwardFunction (reference ops/backward.py:405-455): unpacked
    fc1_1 / fc1_2 [E, F, H] and fc2 [E, H, F]; gradients flow back to every
    input in those layouts."""
    spec = SMALL[0]
    inp = make_inputs(spec, device="cuda", seed=41, weight_scale=0.1)
    I = spec.inter
    gu = inp["gate_up"]                                     # [E, H, 2I]
    fc1_1 = gu[:, :, :I].transpose(1, 2).contiguous().requires_grad_(True)
    fc1_2 = gu[:, :, I:].transpose(1, 2).contiguous().requires_grad_(True)
    fc2 = inp["down"].contiguous().requires_grad_(True)     # [E, H, I]
    x = inp["x"].clone().requires_grad_(True)
    rw = inp["rw"].clone().requires_grad_(True)
    out = mega_moe.MegaMoEBackwardFunction.apply(x, rw, inp["selected"], fc1_1, fc1_2, fc2, None, spec.top_k,
                                                 torch.empty(1, device="cuda"))
    out.backward(inp["dy"])
    torch.cuda.synchronize()
    ref_out, st = O.forward(inp["x"].cpu(), inp["selected"].cpu(), gu.cpu(), fc2.detach().cpu(), inp["rw"].cpu())
    ref = O.backward(st, inp["dy"].cpu())
    assert_rel(out.detach(), ref_out, 2e-2, "out")
    assert_rel(x.grad, ref["grad_hidden"], 2e-2, "dx")
    assert_rel(rw.grad, ref["grad_routing_weights"], 2e-2, "drw")
    assert_rel(fc1_1.grad, ref["grad_gate_up"][:, :, :I].transpose(1, 2), 2e-2, "dfc1_1")
    assert_rel(fc1_2.grad, ref["grad_gate_up"][:, :, I:].transpose(1, 2), 2e-2, "dfc1_2")
    assert_rel(fc2.grad, ref["grad_fc2"], 2e-2, "dfc2")


@pytest.mark.parametrize("spec", [SMALL[1], CaseSpec("overlap_deep_k", 1024, 512, 256, 8, 4, "zipf", True)],
                         ids=lambda s: s.name)
@pytest.mark.parametrize("fmt", ["bf16", "fp8"])
def test_act_backward_overlap_is_bit_identical(spec, fmt, monkeypatch):
    """Step 2 on a second stream beside step 3 (MM_BWD_ACT_OVERLAP=1, the
    default above 1024 rows per expert) gives the same bits
    as the one-stream order, and the side stream's outputs are complete when
    the backward returns (the FC1 dgrad waits for them)."""
    inp = make_inputs(spec, device="cuda", seed=21)
    op = _op(spec, save_fc1_dtype=fmt)
    got = {}
    for ov in ("0", "1", "0"):
        monkeypatch.setenv("MM_BWD_ACT_OVERLAP", ov)
        out, saved = op.forward(inp["x"], inp["selected"], inp["gate_up"], inp["down"], inp["rw"],
                                return_saved=True)
        g = mega_moe.moe_backward_triton(saved, inp["dy"])
        del saved                                   # the side stream's inputs may be released at once
        scratch = torch.randn(1 << 22, device="cuda")  # allocations right after must not disturb it
        vals = {k: g[k].clone() for k in ("grad_hidden", "grad_routing_weights", "grad_fc2", "grad_gate_up",
                                           "grad_fc1_output", "grad_gate")}
        del scratch
        if ov in got:
            for k, v in vals.items():
                assert torch.equal(v, got[ov][k]), k
        got[ov] = vals
    for k in got["0"]:
        assert torch.equal(got["0"][k], got["1"][k]), f"{k} differs with the overlapped activation backward"


def test_stage_timing_environment(monkeypatch):
    """MOE_FWD_TIMING=1 attaches a stage timer to a new operator;
    MOE_BWD_STAGE_TIMING=1 appends each backward's [dispatch, fc2_wgrad,
    swiglu, fc1_wgrad, combine] milliseconds to saved["_bwd_stage_samples"]
    (reference ops/backward.py:216-230, 333-347)."""
    spec = SMALL[0]
    inp = make_inputs(spec, device="cuda", seed=9)
    monkeypatch.setenv("MOE_FWD_TIMING", "1")
    monkeypatch.setenv("MOE_BWD_STAGE_TIMING", "1")
    op = _op(spec)
    assert op.stage_timer is not None
    op.stage_timer = None                      # the backward then times itself
    for overlap in ("0", "1", "0"):
        # with the activation backward on the second stream its time is part
        # of fc2_wgrad and the swiglu interval is NaN (not a stale value)
        monkeypatch.setenv("MM_BWD_ACT_OVERLAP", overlap)
        out, saved = op.forward(inp["x"], inp["selected"], inp["gate_up"], inp["down"], inp["rw"],
                                return_saved=True)
        mega_moe.moe_backward_triton(saved, inp["dy"])
        samples = saved["_bwd_stage_samples"]
        assert len(samples) == 1 and len(samples[0]) == 5
        d, w2, sw, w1, c = samples[0]
        assert all(v > 0 for v in (d, w2, w1, c))
        assert (math.isnan(sw) if overlap == "1" else sw > 0)


def test_stage_timing_sync_finalize():
    from mega_moe.runtime.timing import StageTimer

    spec = SMALL[0]
    inp = make_inputs(spec, device="cuda", seed=9)
    op = _op(spec)
    op.stage_timer = StageTimer()
    out = op.forward(inp["x"], inp["selected"], inp["gate_up"], inp["down"], inp["rw"])
    op.sync()
    t = op.read_last_forward_phase_timing()
    assert {"route", "fc1_swiglu", "fc2", "combine"} <= set(t) and all(v > 0 for v in t.values())
    op.finalize()
    assert out.shape == inp["x"].shape
