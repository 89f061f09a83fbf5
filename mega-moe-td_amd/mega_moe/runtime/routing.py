"""Routing plan on one MI355X.

``MoERoutingPlan`` keeps the reference's field names and meaning
(src/mega_moe/runtime/routing.py:21-54). With one GPU the expert-parallel
world size is 1, so every "send" table equals the "receive" table and both
are expert-major: row i of the dispatched buffer holds flat route
``send_route_indices[i]`` (= token * top_k + slot), rows of one expert are
contiguous and in ascending route order (a stable sort by expert id).

The plan is computed by ``mm_route`` (one device pass, no sort); only
``build_routing_plan`` reads the valid-route count back to the host, as the
reference's builder does (routing.py:636-637, :734). The fused forward and
backward never build a plan and never synchronise.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from .. import _lib


@dataclass
class MoERoutingPlan:
    """Single-in-flight routing metadata shared by dispatch and combine."""

    num_input_tokens: int
    num_received_routes: int
    selected_experts: torch.Tensor
    send_token_indices: torch.Tensor
    send_bucket_starts: torch.Tensor
    send_bucket_receive_offsets: torch.Tensor
    send_counts_by_rank_expert: torch.Tensor
    num_sent_routes: int
    received_routes_per_expert: torch.Tensor
    received_expert_offsets: torch.Tensor
    receive_counts_by_source_expert: torch.Tensor
    stable_sort_indices: torch.Tensor
    valid_route_mask: torch.Tensor
    physical_experts_per_rank: int = 0
    active_physical_experts_per_rank: int = 0
    experts_to_copy: torch.Tensor | None = None
    send_route_indices: torch.Tensor | None = None
    experts_to_copy_cpu: torch.Tensor | None = None
    owner_token: object | None = None
    generation: int = 0
    selected_experts_version: int = -1
    # MI355X additions (appended so positional construction stays valid):
    # inverse permutation [T*k] (-1 = dropped), as build_route_to_send
    # (kernels/fc2_combine.py:508-529) produces it.
    route_to_send: torch.Tensor | None = None


class RouteTables:
    """Device-resident routing tables of one pass (capacity T*k rows)."""

    __slots__ = ("counts", "offsets", "send_route", "send_token", "route_to_send", "weight_perm",
                 "num_routes", "num_experts", "top_k")

    def __init__(self, num_routes: int, num_experts: int, top_k: int, device, with_weights: bool):
        i32 = dict(dtype=torch.int32, device=device)
        self.num_routes = num_routes
        self.num_experts = num_experts
        self.top_k = top_k
        self.counts = torch.empty(num_experts, **i32)
        self.offsets = torch.empty(num_experts + 1, **i32)
        self.send_route = torch.empty(num_routes, **i32)
        self.send_token = torch.empty(num_routes, **i32)
        self.route_to_send = torch.empty(num_routes, **i32)
        self.weight_perm = (torch.empty(num_routes, dtype=torch.float32, device=device)
                            if with_weights else None)


def route(selected_experts: torch.Tensor, num_experts: int, routing_weights: Optional[torch.Tensor],
          workspace: torch.Tensor) -> RouteTables:
    """Launch ``mm_route`` on the current stream; returns device tables."""
    num_routes = selected_experts.numel()
    top_k = selected_experts.shape[1]
    device = selected_experts.device
    tables = RouteTables(num_routes, num_experts, top_k, device, routing_weights is not None)
    need = int(_lib.load().mm_route_workspace_bytes(num_routes, num_experts))
    if workspace.numel() < need:
        raise ValueError(f"routing workspace holds {workspace.numel()} bytes, needs {need}")
    _lib.call(
        "mm_route", _lib.ptr(selected_experts), num_routes, top_k, num_experts, _lib.ptr(routing_weights),
        _lib.ptr(tables.counts), _lib.ptr(tables.offsets), _lib.ptr(tables.send_route),
        _lib.ptr(tables.send_token), _lib.ptr(tables.route_to_send), _lib.ptr(tables.weight_perm),
        _lib.ptr(workspace), workspace.numel(), _lib.stream_of(device))
    return tables


def plan_from_tables(tables: RouteTables, selected_experts: torch.Tensor) -> MoERoutingPlan:
    """Materialise a ``MoERoutingPlan`` (one host read of the valid count)."""
    num_experts = tables.num_experts
    num_valid = int(tables.offsets[num_experts].item())
    flat = selected_experts.reshape(-1)
    valid = (flat >= 0) & (flat < num_experts)
    send_route = tables.send_route[:num_valid]
    # rank of each route among the valid routes -> index into the kept list
    valid_rank = torch.cumsum(valid.to(torch.int64), 0) - 1
    stable_sort_indices = valid_rank[send_route.to(torch.int64)]
    counts = tables.counts
    starts = tables.offsets[:num_experts]
    return MoERoutingPlan(
        num_input_tokens=selected_experts.shape[0],
        num_received_routes=num_valid,
        selected_experts=selected_experts,
        send_token_indices=tables.send_token[:num_valid],
        send_bucket_starts=starts,
        send_bucket_receive_offsets=starts,
        send_counts_by_rank_expert=counts.view(1, num_experts),
        num_sent_routes=num_valid,
        received_routes_per_expert=counts,
        received_expert_offsets=tables.offsets,
        receive_counts_by_source_expert=counts.view(1, num_experts),
        stable_sort_indices=stable_sort_indices,
        valid_route_mask=valid,
        physical_experts_per_rank=num_experts,
        active_physical_experts_per_rank=num_experts,
        experts_to_copy=None,
        send_route_indices=send_route,
        route_to_send=tables.route_to_send,
    )


__all__ = ["MoERoutingPlan", "RouteTables", "route", "plan_from_tables"]
