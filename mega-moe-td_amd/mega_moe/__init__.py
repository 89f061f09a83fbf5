"""MI355X-native Mega-MoE: public API (names of src/mega_moe/__init__.py:1-27)."""

from .config import MoEForwardConfig
from .ops.backward import MegaMoEBackwardFunction, moe_backward_triton
from .ops.forward import DispatchFC1Result, FusedMoEForward, pack_gate_up_weights
from .ops.function import MegaMoEFunction
from .runtime.routing import MoERoutingPlan

__all__ = [
    "FusedMoEForward",
    "DispatchFC1Result",
    "pack_gate_up_weights",
    "MegaMoEBackwardFunction",
    "MegaMoEFunction",
    "moe_backward_triton",
    "MoEForwardConfig",
    "MoERoutingPlan",
]
