"""MegaMoEFunction: the autograd entry of the fused operator.

Follows src/mega_moe/ops/function.py:41-222: ``forward`` runs
``FusedMoEForward.forward(..., return_saved=True)`` and keeps the saved dict
on ctx; ``backward`` checks the owner/generation gates, runs the five-stage
backward and returns the packed ``[E, H, 2F]`` gate/up gradient.

On one GPU ``peer_mem`` has no role (there is no symmetric heap); it must
still not be ``None``, as in the reference, and any tensor may be passed.
``state`` is accepted and left untouched: the MI355X backward keeps no
cross-step state.
"""

import torch

from .backward import moe_backward_triton


class MegaMoEFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, op, hidden_states, routing_weights, selected_experts, gate_up_weight, down_weight, peer_mem,
                state):
        if peer_mem is None:
            raise ValueError(
                "peer_mem must be passed explicitly (any placeholder tensor on one GPU)")
        with torch.no_grad():
            output, saved = op.forward(hidden_states, selected_experts, gate_up_weight, down_weight,
                                       routing_weights, return_saved=True)
        ctx.op = op
        ctx.saved = saved
        ctx.state = state
        return output

    @staticmethod
    def backward(ctx, dy):
        op = ctx.op
        saved = ctx.saved
        if saved.get("_owner_token") != id(op._routing_owner_token):
            raise RuntimeError(
                "the saved dict belongs to another operator instance; run the forward and backward "
                "on the same operator")
        if saved.get("_routing_generation") != op._routing_generation and not saved.get("_single_kernel_snapshot"):
            raise RuntimeError(
                "the saved dict belongs to a routing plan this operator has already superseded; run "
                "backward before the next forward on the operator")
        grads = moe_backward_triton(saved, dy)
        return (None, grads["grad_hidden"], grads["grad_routing_weights"], None, grads["grad_gate_up"],
                grads["grad_fc2"], None, None)


__all__ = ["MegaMoEFunction"]
