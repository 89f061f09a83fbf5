"""The saved dict against the reference's native saved-contract checks (GPU).

Mirrors tests/layer/test_moe_suite.py:3092-3200 of the reference on one GPU:
the bitwise metadata keys (tile tables rebuilt by a per-tile loop, as the
reference's replay builder does), the send-order permutation against an
independent stable argsort of the router output, the permutation pairs, the
host scalars, and the zero-copy weight views (aliasing the inputs, exact
inverses of ``pack_gate_up_weights``).
"""

import pytest
import torch

import mega_moe
from mega_moe.bench_configs import CaseSpec, make_inputs

pytestmark = pytest.mark.gpu

BITWISE_KEYS = ("expert_counts", "split_size_cum_per_expert", "meta_expert_ids", "meta_split_cum", "meta_tile_num",
                "meta_tile_num_cum", "num_tiles_total", "selected_experts")
SCALAR_KEYS = ("batch_size", "hidden_dim", "ffn_dim", "topk", "world_size", "ep_rank", "experts_per_rank", "M",
               "total_send", "total_recv", "splits_send_list", "splits_recv_list")
VIEW_KEYS = ("fc1_1", "fc1_2", "fc1_combined", "fc2")


def _tile_tables(counts, block=64):
    """Per-tile loop (the reference replay builder's form)."""
    ids, split, num, num_cum = [], [], [], []
    tok = tile = 0
    for e, c in enumerate(counts):
        n = (c + block - 1) // block
        for t in range(n):
            ids.append(e)
            split.append(tok)
            num.append(t)
            num_cum.append(tile)
        tok += c
        tile += n
    return ids, split, num, num_cum, tile


@pytest.mark.parametrize("drops", [False, True])
def test_saved_contract(drops):
    spec = CaseSpec("saved", 300, 256, 256, 12, 4, "softmax_topk", True)
    inp = make_inputs(spec, device="cuda", seed=21, weight_scale=0.1)
    sel = inp["selected"].clone()
    if drops:
        sel[0, 0] = -1
        sel[7, 2] = spec.experts + 2
        sel[100, :] = -1
    op = mega_moe.FusedMoEForward(None, max_tokens_per_rank=spec.tokens, hidden_size=spec.hidden,
                                  top_k=spec.top_k, num_experts=spec.experts)
    out, saved = op.forward(inp["x"], sel, inp["gate_up"], inp["down"], inp["rw"], return_saved=True)
    torch.cuda.synchronize()
    E, F = spec.experts, spec.inter
    flat = sel.reshape(-1).to(torch.int64).cpu()
    valid = (flat >= 0) & (flat < E)
    nv = int(valid.sum())

    for key in BITWISE_KEYS + SCALAR_KEYS + VIEW_KEYS + ("sort_idxs", "inv_sort", "local_sort_idxs", "inv_local"):
        assert key in saved, key

    # bitwise metadata
    counts = torch.bincount(flat[valid], minlength=E)
    assert torch.equal(saved["expert_counts"].cpu().to(torch.int64), counts)
    assert saved["split_size_cum_per_expert"].cpu().tolist() == [0] + counts.cumsum(0).tolist()
    ids, split, num, num_cum, ntiles = _tile_tables(counts.tolist())
    assert saved["meta_expert_ids"].cpu().tolist() == ids
    assert saved["meta_split_cum"].cpu().tolist() == split
    assert saved["meta_tile_num"].cpu().tolist() == num
    assert saved["meta_tile_num_cum"].cpu().tolist() == num_cum
    assert saved["num_tiles_total"].cpu().tolist() == [ntiles]
    assert saved["selected_experts"] is sel

    # host values
    assert saved["M"] == saved["total_recv"] == saved["total_send"] == nv
    assert saved["splits_send_list"] == saved["splits_recv_list"] == [nv]
    assert (saved["world_size"], saved["ep_rank"], saved["experts_per_rank"]) == (1, 0, E)

    # send order: stable sort of the valid routes by expert (independent oracle)
    order = torch.argsort(flat.to(torch.float32), stable=True)
    expect = order[valid[order]]
    sort_idxs = saved["sort_idxs"].cpu()
    assert torch.equal(sort_idxs, expect)
    inv_sort = saved["inv_sort"].cpu()
    assert torch.equal(sort_idxs[inv_sort], torch.sort(sort_idxs).values)
    if not drops:
        assert torch.equal(inv_sort[sort_idxs], torch.arange(nv))
    assert torch.equal(saved["local_sort_idxs"].cpu(), torch.arange(nv))
    assert torch.equal(saved["inv_local"].cpu()[saved["local_sort_idxs"].cpu()], torch.arange(nv))
    assert torch.equal(saved["forward_send_route"].cpu().to(torch.int64), expect)

    # activations keyed like the reference's H2 section
    x = inp["x"].cpu()
    assert torch.equal(saved["recv_hidden_sorted"].cpu(), x[expect // spec.top_k])
    assert torch.equal(saved["recv_weights_sorted"][:nv].cpu(), inp["rw"].reshape(-1).cpu()[expect])

    # zero-copy weight views
    w1 = inp["gate_up"]
    for key in ("fc1_1", "fc1_2", "fc1_combined"):
        assert saved[key].untyped_storage().data_ptr() == w1.untyped_storage().data_ptr(), key
    assert saved["fc2"] is inp["down"]
    assert tuple(saved["fc1_combined"].shape) == (E, 2 * F, spec.hidden)
    repacked = mega_moe.pack_gate_up_weights(saved["fc1_1"].contiguous(), saved["fc1_2"].contiguous())
    assert torch.equal(repacked, w1)

    # the backward runs unchanged on the enriched dict
    g = mega_moe.moe_backward_triton(saved, inp["dy"], peer_mem=None)
    torch.cuda.synchronize()
    assert torch.isfinite(g["grad_hidden"].float()).all()
