"""FusedMoEForward on one MI355X.

Public surface and validation follow the reference operator
(src/mega_moe/ops/forward.py): constructor :78-243, ``build_routing_plan``
:853-884, ``dispatch_fc1`` :928-1320, ``forward`` :1884-2109, validators
:766-850, ``pack_gate_up_weights`` :2112-2137, ``DispatchFC1Result`` :57-65.

Pipeline of ``forward`` (all on the caller's stream, no host sync):

    mm_route       selected_experts -> expert-major tables + permuted weights
    mm_fc1_swiglu  rows gathered from hidden_states by send_token (the
                   one-GPU dispatch is fused into the A-tile load) @ W1[e],
                   weighted gated activation in the epilogue -> act [R, I]
    mm_grouped_gemm act @ down[e]^T -> y [R, H]
    mm_combine     out[t] = sum_j y[route_to_send[t*k+j]]  (fp32, slot order)

Every intermediate is sized by the route capacity R = T*k; rows past the
valid count are never read.
"""

from __future__ import annotations

import os

from dataclasses import dataclass
from typing import Optional

import torch
import torch.distributed

from ..config import MoEForwardConfig
from ..runtime.routing import MoERoutingPlan, RouteTables, plan_from_tables, route
from ._saved import MoESaved
from ..runtime.timing import NULL_TIMER, StageTimer
from . import _kernels as K

# Device-kernel limits (csrc/routing.hip kMaxExperts, csrc/rowops.hip combine slots).
MAX_EXPERTS = 32768
MAX_TOP_K = 64


@dataclass
class DispatchFC1Result:
    """Outputs and route identity produced by the dispatch plus FC1 stage."""

    routing_plan: MoERoutingPlan
    fc1_output: torch.Tensor
    dispatched_tokens: torch.Tensor
    received_routing_weights: torch.Tensor
    send_route_indices: torch.Tensor


class FusedMoEForward(torch.nn.Module):
    """BF16 post-routing MoE forward (routing -> FC1+act -> FC2 -> combine).

    ``ep_group`` may be ``None`` (single GPU). All experts live on this GPU;
    an expert-parallel group of size > 1 is rejected because cross-GPU
    dispatch is not part of this build.
    """

    def __init__(
        self,
        ep_group: Optional[torch.distributed.ProcessGroup],
        *,
        max_tokens_per_rank: int,
        hidden_size: int,
        top_k: int,
        num_experts: int,
        config: Optional[MoEForwardConfig] = None,
    ):
        super().__init__()
        if max_tokens_per_rank <= 0:
            raise ValueError("max_tokens_per_rank must be positive")
        if hidden_size <= 0:
            raise ValueError("hidden_size must be positive")
        if top_k <= 0:
            raise ValueError("top_k must be positive")
        if num_experts <= 0:
            raise ValueError("num_experts must be positive")
        if num_experts > MAX_EXPERTS:
            raise ValueError(f"num_experts must be <= {MAX_EXPERTS} (the routing kernel's per-expert tables), "
                             f"got {num_experts}")
        if top_k > MAX_TOP_K:
            raise ValueError(f"top_k must be <= {MAX_TOP_K} (the combine kernel's slot limit), got {top_k}")
        if config is not None and not isinstance(config, MoEForwardConfig):
            raise TypeError("config must be a MoEForwardConfig instance or None")

        self.ep_group = ep_group
        if ep_group is not None:
            self.rank, self.world_size = ep_group.rank(), ep_group.size()
        elif torch.distributed.is_available() and torch.distributed.is_initialized():
            self.rank, self.world_size = torch.distributed.get_rank(), torch.distributed.get_world_size()
        else:
            self.rank, self.world_size = 0, 1
        if num_experts % self.world_size:
            raise ValueError("num_experts must be divisible by the EP world size")
        if self.world_size != 1:
            raise NotImplementedError(
                "expert-parallel dispatch across GPUs is not built; run one operator per GPU "
                "with all experts resident (ep world size 1)")

        self.max_tokens_per_rank = max_tokens_per_rank
        self.hidden_size = hidden_size
        self.top_k = top_k
        self.num_experts = num_experts
        self.experts_per_rank = num_experts // self.world_size
        self.activation_dtype = torch.bfloat16
        self.config = config if config is not None else MoEForwardConfig()
        if self.config.enable_moonep:
            raise NotImplementedError("MoonEP replica balancing is multi-GPU and not built")
        if self.config.save_fc1_dtype == "fp8" and self.config.fc1_gemm_block_size_n != 256:
            # the FP8 save carries one scale per fc1_gemm_block_size_n // 2 columns; the
            # device kernels fix that group at 128 (the reference default block of 256)
            raise NotImplementedError("save_fc1_dtype='fp8' is built for fc1_gemm_block_size_n=256 "
                                      "(128-column scale groups)")
        self.enable_moonep = False
        self.enable_single_kernel_forward = self.config.enable_single_kernel_forward
        self.physical_experts_per_rank = self.experts_per_rank
        self.activation = self.config.activation
        self.situ_beta = self.config.situ_beta
        self.situ_linear_beta = self.config.situ_linear_beta
        self.clamp_limit = self.config.clamp_limit

        self._routing_owner_token = object()
        self._routing_generation = 0
        self._forward_stream = None
        self._device = None
        # optional runtime.timing.StageTimer: HIP events between stages
        # (MOE_FWD_TIMING=1 attaches one, as the reference's phase stamps are
        # switched on by that variable, ops/forward.py:1656-1660)
        self.stage_timer = StageTimer() if os.environ.get("MOE_FWD_TIMING", "0") == "1" else None
        # operator-owned workspaces (routing scratch, tile lists, weight-gradient
        # operand staging), sized for max_tokens_per_rank at the first forward so
        # that they never move afterwards (a captured graph keeps their addresses)
        self._workspaces = K.WorkspacePool()
        self._ws_ready = False

    # ------------------------------------------------------------ validation
    def _check_device(self, t: torch.Tensor, name: str):
        if t.device.type != "cuda":
            raise ValueError(f"{name} must be on the operator's HIP device")
        if self._device is None:
            self._device = t.device
        elif t.device != self._device:
            raise ValueError(f"{name} must be on the operator's HIP device")

    def _validate_topk_indices(self, selected_experts: torch.Tensor):
        if selected_experts.ndim != 2:
            raise ValueError(
                f"selected_experts must have shape [tokens, top_k], got {tuple(selected_experts.shape)}")
        if selected_experts.shape[1] != self.top_k:
            raise ValueError(
                f"selected_experts must have top_k={self.top_k}, got shape {tuple(selected_experts.shape)}")
        if selected_experts.dtype != torch.int32:
            raise TypeError(f"selected_experts must use torch.int32, got {selected_experts.dtype}")
        self._check_device(selected_experts, "selected_experts")
        if not selected_experts.is_contiguous():
            raise ValueError("selected_experts must be contiguous")
        if selected_experts.shape[0] > self.max_tokens_per_rank:
            raise ValueError(
                f"input has {selected_experts.shape[0]} tokens, exceeding "
                f"max_tokens_per_rank={self.max_tokens_per_rank}")

    def _validate_dispatch_inputs(self, hidden_states: torch.Tensor, selected_experts: torch.Tensor):
        self._validate_topk_indices(selected_experts)
        if hidden_states.ndim != 2:
            raise ValueError(
                f"hidden_states must have shape [tokens, hidden], got {tuple(hidden_states.shape)}")
        expected_shape = (selected_experts.shape[0], self.hidden_size)
        if tuple(hidden_states.shape) != expected_shape:
            raise ValueError(f"hidden_states must have shape {expected_shape}, got {tuple(hidden_states.shape)}")
        if hidden_states.dtype != self.activation_dtype:
            raise TypeError(f"hidden_states must use {self.activation_dtype}, got {hidden_states.dtype}")
        if hidden_states.device != selected_experts.device:
            raise ValueError("hidden_states and selected_experts must be on the same device")
        if not hidden_states.is_contiguous():
            raise ValueError("hidden_states must be contiguous")

    def _validate_gate_up_weight(self, gate_up_weight: torch.Tensor, device: torch.device):
        if gate_up_weight.ndim != 3:
            raise ValueError("gate_up_weight must have shape [experts_per_rank, hidden, 2F]")
        if gate_up_weight.shape[0] != self.experts_per_rank:
            raise ValueError(
                f"gate_up_weight has {gate_up_weight.shape[0]} local experts, expected {self.experts_per_rank}")
        if gate_up_weight.shape[1] != self.hidden_size:
            raise ValueError(
                "gate_up_weight must use [experts_per_rank, hidden, 2F] layout "
                f"with hidden_size={self.hidden_size}, got {tuple(gate_up_weight.shape)}")
        packed_output_size = gate_up_weight.shape[2]
        if packed_output_size <= 0 or packed_output_size % 2:
            raise ValueError("gate_up_weight output dimension must be a positive even value (2F)")
        if gate_up_weight.dtype != self.activation_dtype:
            raise TypeError(f"gate_up_weight must use {self.activation_dtype}, got {gate_up_weight.dtype}")
        if gate_up_weight.device != device:
            raise ValueError("gate_up_weight and hidden_states must be on the same device")
        if not gate_up_weight.is_contiguous():
            raise ValueError("gate_up_weight must be contiguous and pre-packed before forward")

    def _validate_routing_weights(self, routing_weights, selected_experts):
        if (routing_weights.shape != selected_experts.shape or routing_weights.dtype != torch.float32
                or routing_weights.device != selected_experts.device or not routing_weights.is_contiguous()):
            raise ValueError(
                "routing_weights must be contiguous FP32 with the same shape and device as selected_experts")

    def _validate_down_weight(self, down_weight, gate_up_weight, device):
        expected = (self.experts_per_rank, self.hidden_size, gate_up_weight.shape[2] // 2)
        if (down_weight.ndim != 3 or tuple(down_weight.shape) != expected
                or down_weight.dtype != self.activation_dtype or down_weight.device != device):
            raise ValueError(
                f"down_weight must be BF16 with shape {expected} on the input device (a strided "
                "natural-layout [E, F, H] view flows through unstaged)")
        se, sh, sf = down_weight.stride()
        if not (sf == 1 or sh == 1):
            raise ValueError("down_weight must be contiguous along hidden or ffn (a [E,H,F] table or "
                             "the transposed view of an [E,F,H] table)")

    def _validate_tiles(self, gate_up_weight):
        ffn_size = gate_up_weight.shape[2] // 2
        cfg = self.config
        if (gate_up_weight.shape[2] % cfg.fc1_gemm_block_size_n or self.hidden_size % cfg.fc1_gemm_block_size_k
                or self.hidden_size % cfg.fc2_gemm_block_size_n or ffn_size % cfg.fc2_gemm_block_size_k):
            raise ValueError("configured FC1/FC2 N and K tiles must divide the weight dimensions")
        # MI355X kernel tiles: 128-wide N/M tiles, 64-deep K steps.
        if self.hidden_size % 128 or ffn_size % 128:
            raise ValueError("hidden_size and ffn size must be multiples of 128 for the MFMA tiles")

    def _check_stream(self, device):
        current = torch.cuda.current_stream(device)
        if self._forward_stream is None:
            self._forward_stream = current
        elif self._forward_stream != current:
            raise RuntimeError(
                "FusedMoEForward is single-stream; recreate the operator for a different caller stream")

    # ------------------------------------------------------------ lifecycle
    def sync(self):
        """Wait for the work queued on the current device (reference ops/forward.py:284-285)."""
        torch.cuda.synchronize()

    def finalize(self):
        """Drain queued work and release the operator's workspaces (reference
        ops/forward.py:287-300). One GPU holds no symmetric memory or
        transport streams; graphs captured over this operator must not be
        replayed after finalize()."""
        torch.cuda.synchronize()
        self._workspaces.release()
        self._ws_ready = False

    def read_last_forward_phase_timing(self):
        """Mean per-stage milliseconds of the passes recorded by the attached
        ``runtime.timing.StageTimer`` (``op.stage_timer``), the HIP-event
        counterpart of the reference's single-kernel phase stamps
        (ops/forward.py:1555-1570). Synchronises. Raises ``RuntimeError``
        when no timer is attached, as the reference does before any timed
        forward has run."""
        if self.stage_timer is None:
            raise RuntimeError("no stage timer is attached to this operator; set op.stage_timer = StageTimer()")
        return self.stage_timer.summary()

    def lend_replica_weight_tables_for_grad(self, *, experts_to_copy_cpu=None):
        """MoonEP replica tables (reference ops/forward.py:1322) do not exist
        on one GPU: expert parallelism and MoonEP are not built."""
        raise NotImplementedError("MoonEP replica weight tables are not built (one GPU, no expert parallelism)")

    @property
    def max_routes(self) -> int:
        return self.max_tokens_per_rank * self.top_k

    def _reserve_workspaces(self, device):
        """Size the routing and tile-list workspaces for the operator's capacity."""
        if self._ws_ready:
            return
        R, E = self.max_routes, self.experts_per_rank
        self._workspaces.get(device, K.route_workspace_bytes(R, E), "route")
        self._workspaces.get(device, K.gemm_workspace_bytes(R, E), "gemm")
        self._ws_ready = True

    def _route(self, selected_experts, routing_weights) -> RouteTables:
        self._reserve_workspaces(selected_experts.device)
        num_routes = selected_experts.numel()
        need = K.route_workspace_bytes(num_routes, self.experts_per_rank)
        ws = self._workspaces.get(selected_experts.device, need, "route")
        return route(selected_experts, self.experts_per_rank, routing_weights, ws)

    # ------------------------------------------------------------ routing
    def build_routing_plan(self, selected_experts: torch.Tensor, *, moonep_plan_hook=None) -> MoERoutingPlan:
        """Build stable dispatch/count metadata for one set of selected experts."""
        self._validate_topk_indices(selected_experts)
        if moonep_plan_hook is not None:
            raise NotImplementedError("MoonEP planning is not built")
        self._routing_generation += 1
        tables = self._route(selected_experts, None)
        plan = plan_from_tables(tables, selected_experts)
        plan.owner_token = self._routing_owner_token
        plan.generation = self._routing_generation
        plan.selected_experts_version = selected_experts._version
        return plan

    # ------------------------------------------------------------ dispatch + FC1
    def dispatch_fc1(self, hidden_states, selected_experts, routing_plan: MoERoutingPlan, fc1_weight,
                     fc1_output=None, *, routing_weights, **unsupported) -> DispatchFC1Result:
        """Dispatch (local gather) and the raw FC1 GEMM of the staged path.

        ``fc1_weight`` is the contiguous ``[E, K=H, N]`` table; the result's
        ``fc1_output`` is ``dispatched_tokens @ fc1_weight[e]`` per row in bf16
        (reference forward.py:928-1320; MoonEP arguments are rejected).
        """
        if any(v is not None for v in unsupported.values()):
            raise NotImplementedError(f"unsupported dispatch_fc1 arguments: {sorted(unsupported)}")
        self._validate_dispatch_inputs(hidden_states, selected_experts)
        if routing_plan.selected_experts is not selected_experts:
            raise ValueError("routing_plan must be built from this exact selected_experts tensor")
        if routing_plan.num_input_tokens != hidden_states.shape[0]:
            raise ValueError("routing plan token count does not match hidden_states")
        if fc1_weight.ndim != 3:
            raise ValueError("fc1_weight must be a 3D local-expert weight tensor")
        if fc1_weight.shape[0] != self.experts_per_rank:
            raise ValueError(
                f"fc1_weight has {fc1_weight.shape[0]} local experts, expected {self.experts_per_rank}")
        if fc1_weight.dtype != self.activation_dtype:
            raise TypeError(f"fc1_weight must use {self.activation_dtype}, got {fc1_weight.dtype}")
        if fc1_weight.device != hidden_states.device:
            raise ValueError("fc1_weight and hidden_states must be on the same device")
        if fc1_weight.shape[1] != self.hidden_size:
            raise ValueError(
                "fc1_weight must use [experts_per_rank, hidden_size, output_size] "
                f"layout, got {tuple(fc1_weight.shape)}")
        if fc1_weight.shape[2] <= 0 or fc1_weight.shape[2] % 128:
            raise ValueError("fc1_weight output_size must be a positive multiple of 128")
        if not fc1_weight.is_contiguous():
            raise ValueError("fc1_weight must be contiguous in [expert, K, N] layout")
        if routing_weights.shape != selected_experts.shape:
            raise ValueError("routing_weights must match selected_experts shape [tokens, top_k]")
        if routing_weights.dtype != torch.float32:
            raise TypeError(f"routing_weights must use torch.float32, got {routing_weights.dtype}")
        if routing_weights.device != hidden_states.device:
            raise ValueError("routing_weights and hidden_states must be on the same device")
        if not routing_weights.is_contiguous():
            raise ValueError("routing_weights must be contiguous")
        m = routing_plan.num_received_routes
        output_size = fc1_weight.shape[2]
        if fc1_output is not None:
            if tuple(fc1_output.shape) != (m, output_size):
                raise ValueError(f"fc1_output must have shape {(m, output_size)}, got {tuple(fc1_output.shape)}")
            if fc1_output.dtype != self.activation_dtype:
                raise TypeError(f"fc1_output must use {self.activation_dtype}, got {fc1_output.dtype}")
            if fc1_output.device != hidden_states.device:
                raise ValueError("fc1_output and hidden_states must be on the same device")
            if not fc1_output.is_contiguous():
                raise ValueError("fc1_output must be contiguous")
        offsets = routing_plan.received_expert_offsets
        dispatched = K.permute(hidden_states, routing_plan.send_token_indices, offsets, m)
        if m:
            gu = K.grouped_gemm(dispatched, None, fc1_weight, fc1_weight.stride(0), 1, fc1_weight.stride(1),
                                offsets, m, output_size, self.hidden_size, pool=self._workspaces)
        else:
            gu = torch.empty(0, output_size, dtype=torch.bfloat16, device=hidden_states.device)
        if fc1_output is not None:
            fc1_output.copy_(gu)
            gu = fc1_output
        received_w = routing_weights.reshape(-1)[routing_plan.send_route_indices.to(torch.int64)]
        return DispatchFC1Result(
            routing_plan=routing_plan,
            fc1_output=gu,
            dispatched_tokens=dispatched,
            received_routing_weights=received_w,
            send_route_indices=routing_plan.send_route_indices,
        )

    # ------------------------------------------------------------ full forward
    def forward(self, hidden_states, selected_experts, gate_up_weight, down_weight, routing_weights, *,
                return_saved: bool = False):
        """Run the complete BF16 post-routing MoE forward.

        With ``return_saved=True`` returns ``(output, saved)``; ``saved`` holds
        the routing tables, the raw FC1 output (``fc1_output`` [R, 2I] =
        [gate | up] bf16), the weighted activation (``swiglu_out_weighted``)
        and references to the inputs; the backward re-gathers dispatched rows
        from ``hidden_states`` instead of keeping a permuted copy.
        """
        self._validate_dispatch_inputs(hidden_states, selected_experts)
        self._validate_gate_up_weight(gate_up_weight, hidden_states.device)
        self._check_stream(hidden_states.device)
        self._validate_routing_weights(routing_weights, selected_experts)
        self._validate_down_weight(down_weight, gate_up_weight, hidden_states.device)
        self._validate_tiles(gate_up_weight)

        num_tokens = hidden_states.shape[0]
        num_routes = num_tokens * self.top_k
        inter = gate_up_weight.shape[2] // 2
        self._routing_generation += 1
        if num_tokens == 0:
            out = torch.empty(0, self.hidden_size, dtype=torch.bfloat16, device=hidden_states.device)
            if not return_saved:
                return out
        tm = self.stage_timer or NULL_TIMER
        tables = None
        if num_tokens:
            tm.begin("route")
            tables = self._route(selected_experts, routing_weights)
            tm.end()
            tm.begin("fc1_swiglu")
            act, fc1_out, fc1_scale = K.fc1_swiglu(
                hidden_states, tables.send_token, gate_up_weight, tables.offsets, tables.weight_perm, num_routes,
                self.activation, self.situ_beta, self.situ_linear_beta, self.clamp_limit, save_fc1=return_saved,
                fc1_dtype=self.config.save_fc1_dtype, pool=self._workspaces)
            tm.end()
            tm.begin("fc2")
            se, sh, sf = down_weight.stride()
            y = K.grouped_gemm(act, None, down_weight, se, sh, sf, tables.offsets, num_routes, self.hidden_size,
                               inter, pool=self._workspaces)
            tm.end()
            tm.begin("combine")
            out = K.combine(y, tables.route_to_send, num_tokens, self.top_k)
            tm.end()
        if not return_saved:
            return out
        saved = MoESaved(
            batch_size=num_tokens, hidden_dim=self.hidden_size, ffn_dim=inter, num_experts=self.num_experts,
            experts_per_rank=self.experts_per_rank, topk=self.top_k, world_size=1, ep_rank=0,
            ep_group=self.ep_group, total_routes=num_routes,
            activation=self.activation, situ_beta=self.situ_beta, situ_linear_beta=self.situ_linear_beta,
            clamp_limit=self.clamp_limit,
            hidden_states=hidden_states, selected_experts=selected_experts, routing_weights=routing_weights,
            gate_up_weight=gate_up_weight, down_weight=down_weight, fc2=down_weight,
            _owner_token=id(self._routing_owner_token), _routing_generation=self._routing_generation,
            _single_kernel_snapshot=bool(self.enable_single_kernel_forward), _stage_timer=self.stage_timer,
            _workspaces=self._workspaces, _max_routes=self.max_routes,
        )
        if tables is not None:
            saved.update(
                expert_counts=tables.counts, split_size_cum_per_expert=tables.offsets,
                send_route_indices=tables.send_route, send_token_indices=tables.send_token,
                route_to_send=tables.route_to_send, recv_weights_sorted=tables.weight_perm,
                fc1_output=fc1_out, swiglu_out_weighted=act,
            )
            if saved_recompute():
                # MOE_SAVED_RECOMPUTE=1 (reference kernels/mega_bwd.py:3208-3226): the backward
                # recomputes act from fc1_output, so the saved dict does not pin it
                del saved["swiglu_out_weighted"]
            if fc1_scale is not None:
                # FP8 save (reference ops/forward.py:1874-1880): one fp32 scale per row and
                # per 128-column group, gate groups then up groups
                saved.update(fc1_output_scale=fc1_scale, fc1_scale_group_size=128)
        return out, saved


def saved_recompute() -> bool:
    """``MOE_SAVED_RECOMPUTE=1``: the backward recomputes the weighted
    activation from ``fc1_output`` instead of reading a saved copy."""
    return os.environ.get("MOE_SAVED_RECOMPUTE", "0") == "1"


def pack_gate_up_weights(gate_weight_local: torch.Tensor, up_weight_local: torch.Tensor) -> torch.Tensor:
    """Pack local BF16 gate/up projections ``[E, F, H]`` as contiguous ``[E, H, 2F]``."""
    if gate_weight_local.ndim != 3 or up_weight_local.ndim != 3:
        raise ValueError("gate and up weights must have shape [experts_per_rank, ffn_size, hidden_size]")
    if gate_weight_local.shape != up_weight_local.shape:
        raise ValueError(
            f"gate and up weight shapes must match, got {gate_weight_local.shape} and {up_weight_local.shape}")
    if gate_weight_local.dtype != torch.bfloat16 or up_weight_local.dtype != torch.bfloat16:
        raise TypeError("gate and up weights must both use torch.bfloat16")
    if gate_weight_local.device != up_weight_local.device:
        raise ValueError("gate and up weights must be on the same device")
    return torch.cat((gate_weight_local.transpose(1, 2), up_weight_local.transpose(1, 2)), dim=2).contiguous()


__all__ = ["DispatchFC1Result", "FusedMoEForward", "pack_gate_up_weights"]
