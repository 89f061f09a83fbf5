"""Host-side API behaviour of the mega_moe mirror (no GPU needed): the
reference's validation rules and error types (src/mega_moe/config.py:196-386,
ops/forward.py:78-243, 766-850, 2112-2137)."""

import pytest
import torch

import mega_moe
from mega_moe import MoEForwardConfig, pack_gate_up_weights


def test_public_names():
    for name in ("FusedMoEForward", "DispatchFC1Result", "pack_gate_up_weights", "MegaMoEBackwardFunction",
                 "MegaMoEFunction", "moe_backward_triton", "MoEForwardConfig", "MoERoutingPlan"):
        assert hasattr(mega_moe, name)


@pytest.mark.parametrize("kw, exc", [
    (dict(dispatch_fc1_block_size_m=24), ValueError),
    (dict(fc1_gemm_block_size_n=8), ValueError),
    (dict(activation="gelu"), ValueError),
    (dict(situ_beta=0.0), ValueError),
    (dict(situ_beta="1"), TypeError),
    (dict(situ_linear_beta=-1.0), ValueError),
    (dict(clamp_limit=0), ValueError),
    (dict(save_fc1_dtype="fp32"), ValueError),
    (dict(receive_capacity_factor=0.5), ValueError),
    (dict(single_kernel_group_windows=3), ValueError),
    (dict(enable_moonep=1), TypeError),
    (dict(enable_single_kernel_forward=True, fc1_gemm_block_size_m=128), ValueError),
])
def test_config_validation(kw, exc):
    with pytest.raises(exc):
        MoEForwardConfig(**kw)


def test_config_defaults():
    c = MoEForwardConfig()
    assert c.activation == "swiglu" and c.single_kernel_group_windows == 32
    assert c.num_aicore_programs > 0 and c.resolved_receive_capacity_factor(4) == 4.0
    assert MoEForwardConfig(receive_capacity_factor=2).resolved_receive_capacity_factor(8) == 2.0


@pytest.mark.parametrize("kw", [
    dict(max_tokens_per_rank=0), dict(hidden_size=0), dict(top_k=0), dict(num_experts=0)])
def test_constructor_rejects_nonpositive(kw):
    base = dict(max_tokens_per_rank=8, hidden_size=256, top_k=2, num_experts=4)
    base.update(kw)
    with pytest.raises(ValueError):
        mega_moe.FusedMoEForward(None, **base)


@pytest.mark.parametrize("kw", [dict(top_k=65), dict(num_experts=32769)])
def test_constructor_rejects_kernel_limits(kw):
    """Limits of the device kernels are rejected up front, not at the first
    forward (combine slots: top_k <= 64; routing tables: E <= 32768)."""
    base = dict(max_tokens_per_rank=8, hidden_size=256, top_k=2, num_experts=4)
    base.update(kw)
    with pytest.raises(ValueError):
        mega_moe.FusedMoEForward(None, **base)


def test_constructor_type_and_unbuilt_features():
    with pytest.raises(TypeError):
        mega_moe.FusedMoEForward(None, max_tokens_per_rank=8, hidden_size=256, top_k=2, num_experts=4, config={})
    with pytest.raises(NotImplementedError):
        mega_moe.FusedMoEForward(None, max_tokens_per_rank=8, hidden_size=256, top_k=2, num_experts=4,
                                 config=MoEForwardConfig(enable_moonep=True))


def test_pack_gate_up_weights():
    g = torch.randn(3, 5, 7).to(torch.bfloat16)
    u = torch.randn(3, 5, 7).to(torch.bfloat16)
    packed = pack_gate_up_weights(g, u)
    assert packed.shape == (3, 7, 10) and packed.is_contiguous()
    assert torch.equal(packed[:, :, :5], g.transpose(1, 2)) and torch.equal(packed[:, :, 5:], u.transpose(1, 2))
    with pytest.raises(ValueError):
        pack_gate_up_weights(g, u[:, :4])
    with pytest.raises(TypeError):
        pack_gate_up_weights(g.float(), u)
    with pytest.raises(ValueError):
        pack_gate_up_weights(g[0], u[0])


def test_forward_rejects_host_tensors():
    op = mega_moe.FusedMoEForward(None, max_tokens_per_rank=8, hidden_size=256, top_k=2, num_experts=4)
    sel = torch.zeros(8, 2, dtype=torch.int32)
    with pytest.raises(ValueError, match="device"):
        op.build_routing_plan(sel)
    with pytest.raises(TypeError):
        op.build_routing_plan(sel.long())
    with pytest.raises(ValueError, match="top_k"):
        op.build_routing_plan(torch.zeros(8, 3, dtype=torch.int32))
    # reference order (forward.py:766-792): the device check precedes the capacity check
    with pytest.raises(ValueError, match="device"):
        op.build_routing_plan(torch.zeros(9, 2, dtype=torch.int32))


def test_backward_requires_saved_activations():
    with pytest.raises(ValueError, match="fc1_output"):
        mega_moe.moe_backward_triton({}, torch.zeros(1, 1))
    with pytest.raises(NotImplementedError):
        mega_moe.moe_backward_triton({"fc1_output": None}, torch.zeros(1, 1), grad_transport=object())


def test_saved_dict_derives_reference_keys_on_cpu():
    """MoESaved: reference contract keys as closed forms of the stored tables."""
    from mega_moe.ops._saved import MoESaved

    E, k, F, H = 5, 2, 128, 256
    sel = torch.tensor([[0, 3], [3, 1], [-1, 0], [4, 3], [1, 9]], dtype=torch.int32)
    flat = sel.reshape(-1).long()
    valid = (flat >= 0) & (flat < E)
    order = torch.argsort(flat.float(), stable=True)
    send_route = order[valid[order]].int()
    counts = torch.bincount(flat[valid], minlength=E).int()
    offsets = torch.zeros(E + 1, dtype=torch.int32)
    offsets[1:] = counts.cumsum(0)
    w1 = torch.randn(E, H, 2 * F).bfloat16()
    x = torch.randn(5, H).bfloat16()
    s = MoESaved(num_experts=E, experts_per_rank=E, ffn_dim=F, split_size_cum_per_expert=offsets,
                 expert_counts=counts, send_route_indices=send_route, send_token_indices=send_route // k,
                 gate_up_weight=w1, hidden_states=x)
    n = int(valid.sum())
    assert "meta_tile_num" in s and "nonexistent" not in s and s.get("nonexistent") is None
    assert s["total_recv"] == s["M"] == n and s["splits_send_list"] == [n]
    assert s["meta_expert_ids"].tolist() == [e for e in range(E) if counts[e] > 0]  # every count < 64
    assert s["num_tiles_total"].tolist() == [int((counts > 0).sum())]
    assert torch.equal(s["sort_idxs"], send_route.long())
    assert torch.equal(s["sort_idxs"][s["inv_sort"]], torch.sort(send_route.long()).values)
    assert torch.equal(s["recv_hidden_sorted"], x[send_route.long() // k])
    assert s["fc1_combined"].shape == (E, 2 * F, H) and s["fc1_1"].data_ptr() == w1.data_ptr()
    assert torch.equal(s["recv_counts_by_source_expert"], counts.view(1, E))
    with pytest.raises(KeyError):
        s["not_a_key"]


def test_operator_timing_and_moonep_entry_points():
    op = mega_moe.FusedMoEForward(None, max_tokens_per_rank=4, hidden_size=256, top_k=2, num_experts=4)
    with pytest.raises(RuntimeError, match="stage timer"):
        op.read_last_forward_phase_timing()
    with pytest.raises(NotImplementedError, match="MoonEP"):
        op.lend_replica_weight_tables_for_grad()
    assert callable(op.sync) and callable(op.finalize)


def test_backward_validates_dy_and_hidden_states_on_cpu():
    """Host-side checks of moe_backward_triton run before any launch."""
    T, H = 4, 256
    saved = dict(batch_size=T, topk=2, hidden_dim=H, ffn_dim=128, total_routes=8, fc1_output=torch.empty(0),
                 gate_up_weight=None, down_weight=None, split_size_cum_per_expert=None,
                 send_token_indices=None, route_to_send=None, hidden_states=torch.zeros(T, H).bfloat16())
    with pytest.raises(ValueError, match="dy must have shape"):
        mega_moe.moe_backward_triton(saved, torch.zeros(T + 1, H), peer_mem=None)
    with pytest.raises(ValueError, match="hidden_states must be"):
        mega_moe.moe_backward_triton(saved, torch.zeros(T, H), peer_mem=None,
                                     hidden_states=torch.zeros(T, H))  # fp32
    with pytest.raises(ValueError, match="missing fc1_output"):
        mega_moe.moe_backward_triton({}, torch.zeros(T, H), peer_mem=None)
    with pytest.raises(NotImplementedError, match="MoonEP"):
        mega_moe.moe_backward_triton(saved, torch.zeros(T, H), peer_mem=None, grad_transport=object())
