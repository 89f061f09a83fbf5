"""HIP graph capture of the layer (GPU): forward + five-stage backward
captured once and replayed, each replay bit-identical to an eager run on the
same inputs.

The path makes no host synchronisation and records no memset nodes: routing
counts, tile lists and every output are written by kernels, so a caller can
capture a training step. The operator is single-stream (the reference's
rule, forward.py:1929-1936), so the eager warm-up and the capture run on the
same side stream; the backward's own fork of the activation backward onto a
second stream (and its join) is captured with it. Replays alternate with eager work on the same tensors and
with new inputs copied into the captured ones.
"""

import pytest
import torch

import mega_moe
from mega_moe.bench_configs import CaseSpec, make_inputs

pytestmark = pytest.mark.gpu

GRADS = ("grad_hidden", "grad_routing_weights", "grad_fc2", "grad_gate_up")


def _step(op, inp):
    out, saved = op.forward(inp["x"], inp["selected"], inp["gate_up"], inp["down"], inp["rw"], return_saved=True)
    g = mega_moe.moe_backward_triton(saved, inp["dy"], peer_mem=None)
    return [out] + [g[k] for k in GRADS]


@pytest.mark.parametrize("spec", [
    CaseSpec("graph_small", 256, 256, 256, 8, 4, "softmax_topk", True),
    CaseSpec("graph_wide", 512, 1024, 512, 16, 2, "zipf", True),
], ids=lambda s: s.name)
@pytest.mark.parametrize("overlap", ["0", "1"])
def test_captured_step_replays_bit_exact(spec, overlap, monkeypatch):
    # overlap=1: the activation backward forks onto a second stream and joins
    # before the FC1 dgrad, inside the capture
    monkeypatch.setenv("MM_BWD_ACT_OVERLAP", overlap)
    inp = make_inputs(spec, device="cuda", seed=5, weight_scale=0.1)
    alt = make_inputs(spec, device="cuda", seed=6, weight_scale=0.1)
    cfg = mega_moe.MoEForwardConfig()
    op = mega_moe.FusedMoEForward(None, max_tokens_per_rank=spec.tokens, hidden_size=spec.hidden,
                                  top_k=spec.top_k, num_experts=spec.experts, config=cfg)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ref_a = [t.clone() for t in _step(op, inp)]      # eager warm-up: workspaces exist before capture
        ref_b = [t.clone() for t in _step(op, {**inp, **{k: alt[k] for k in ("x", "dy", "selected", "rw")}})]
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        outs = _step(op, inp)
    torch.cuda.synchronize()

    saved_x, saved_dy = inp["x"].clone(), inp["dy"].clone()
    saved_sel, saved_rw = inp["selected"].clone(), inp["rw"].clone()
    for rep in range(4):
        use_b = rep % 2 == 1
        src = alt if use_b else {"x": saved_x, "dy": saved_dy, "selected": saved_sel, "rw": saved_rw}
        for k in ("x", "dy", "selected", "rw"):
            inp[k].copy_(src[k])
        graph.replay()
        torch.cuda.synchronize()
        want = ref_b if use_b else ref_a
        for name, got, exp in zip(("output",) + GRADS, outs, want):
            assert torch.equal(got, exp), f"replay {rep}: {name} differs from the eager result"
        # eager work on the same stream and tensors between replays
        with torch.cuda.stream(side):
            again = _step(op, inp)
        torch.cuda.synchronize()
        for name, got, exp in zip(("output",) + GRADS, again, want):
            assert torch.equal(got, exp), f"eager after replay {rep}: {name} differs"


def test_graphs_of_two_sizes_on_one_stream():
    """Graphs captured for a small and then a large batch on one stream, the
    small one replayed after the large one: the operator's workspaces are
    sized for max_tokens_per_rank before the first capture, so neither graph
    holds a freed workspace address; a direct wrapper call that outgrows the
    module pool retires its old buffer instead of freeing it."""
    from mega_moe.ops import _kernels as K

    spec = CaseSpec("graph_sizes", 512, 256, 256, 8, 4, "softmax_topk", True)
    inp = make_inputs(spec, device="cuda", seed=8, weight_scale=0.1)
    op = mega_moe.FusedMoEForward(None, max_tokens_per_rank=spec.tokens, hidden_size=spec.hidden,
                                  top_k=spec.top_k, num_experts=spec.experts)
    sizes = (64, 512)
    parts = {n: {k: (v[:n].clone() if k in ("x", "dy", "selected", "rw") else v) for k, v in inp.items()}
             for n in sizes}
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        eager = {n: [t.clone() for t in _step(op, parts[n])] for n in sizes}
    torch.cuda.synchronize()
    before = op._workspaces.nbytes()
    graphs, outs = {}, {}
    for n in sizes:                                   # small first, then large
        graphs[n] = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graphs[n], stream=side):
            outs[n] = _step(op, parts[n])
    torch.cuda.synchronize()
    assert op._workspaces.nbytes() == before          # nothing grew under capture
    junk = [torch.full((1 << 20,), 7, dtype=torch.int32, device="cuda") for _ in range(8)]
    for n in (512, 64, 512, 64):
        graphs[n].replay()
        torch.cuda.synchronize()
        for name, got, exp in zip(("output",) + GRADS, outs[n], eager[n]):
            assert torch.equal(got, exp), f"tokens={n}: {name} differs from the eager result"
    del junk
    # module pool: growth retires, never frees
    pool = K.WorkspacePool()
    a = pool.get(torch.device("cuda"), 1024, "t")
    b = pool.get(torch.device("cuda"), 4096, "t")
    assert a.data_ptr() != b.data_ptr() and pool.nbytes() == a.numel() + b.numel()
    pool.release()
    assert pool.nbytes() == 0
