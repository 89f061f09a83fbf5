"""MoEForwardConfig for the MI355X operator.

Mirrors the reference dataclass (src/mega_moe/config.py:95-392): the same
field names, defaults and validation messages, so existing callers construct
it unchanged. What the fields mean on MI355X:

* ``num_aicore_programs`` / ``num_aivector_programs`` are resolved from the
  device (compute-unit count) instead of the Ascend CANN driver
  (reference config.py:37-74).
* ``fc1_gemm_block_size_*`` / ``fc2_*`` / ``dispatch_*`` are validated exactly
  as in the reference (powers of two >= 16; dims must be divisible, checked
  by ``FusedMoEForward.forward``). The HIP kernels pick their own MFMA tiles,
  so these values only constrain shapes, as in the reference; the Ascend
  L0C accumulator caps (config.py:8-22) do not apply to CDNA4 and are not
  enforced.
* ``activation`` / ``situ_beta`` / ``situ_linear_beta`` / ``clamp_limit`` select
  the gated activation fused into the FC1 epilogue and its backward.
* ``save_fc1_dtype`` selects the saved raw FC1 output format: ``"bf16"``,
  ``"fp16"`` (the bf16 values as fp16) or ``"fp8"`` (E4M3 with one fp32 scale
  per row and per 128-column group; needs ``fc1_gemm_block_size_n=256``).
* ``enable_moonep`` and the MoonEP knobs are accepted for source
  compatibility; expert-parallel replica balancing is out of scope on one
  GPU, so ``enable_moonep=True`` raises ``NotImplementedError`` when the
  operator is built.
"""

from dataclasses import dataclass, field
from typing import Optional

_ACTIVATIONS = ("swiglu", "situglu", "clamp_swiglu")

# MI355X: 256 compute units in 8 XCDs; used when no GPU is visible (host tests).
_MI355X_COMPUTE_UNITS = 256


def _detect_compute_units() -> int:
    """Compute units of the current HIP device, or the MI355X count without one."""
    try:
        import torch

        if torch.cuda.is_available():
            return int(torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count)
    except Exception:  # pragma: no cover - torch import problems surface elsewhere
        pass
    return _MI355X_COMPUTE_UNITS


@dataclass(frozen=True)
class MoEForwardConfig:
    """Stage tiling / activation parameters (reference config.py:95-392)."""

    num_aicore_programs: int = field(init=False)
    num_aivector_programs: int = field(init=False)
    receive_capacity_factor: Optional[float] = None
    dispatch_fc1_block_size_m: int = 128
    fc1_gemm_block_size_n: int = 256
    fc1_gemm_block_size_k: int = 128
    fc2_combine_block_size_m: int = 256
    fc2_gemm_block_size_n: int = 256
    fc2_gemm_block_size_k: int = 128
    activation: str = "swiglu"
    situ_beta: float = 1.0
    situ_linear_beta: Optional[float] = None
    clamp_limit: float = 7.0
    fc1_gemm_block_size_m: int = 256
    enable_moonep: bool = False
    moonep_replica_gate_up_chunk_bytes: int = 16 * 1024 * 1024
    moonep_replica_down_chunk_bytes: int = 4 * 1024 * 1024
    moonep_replica_down_early_programs: int = 8
    moonep_replica_down_early_descriptors_per_program: int = 2
    moonep_fused_balanced_count: bool = True
    moonep_fused_route_mapping: bool = True
    moonep_enable_replica_cache: bool = True
    enable_single_kernel_forward: bool = False
    save_fc1_dtype: str = "bf16"
    moonep_udma_chunk_bytes: int = 64 * 1024 * 1024
    single_kernel_group_windows: Optional[int] = None
    single_kernel_dispatch_block_size_m: Optional[int] = 256

    def __post_init__(self):
        cus = _detect_compute_units()
        object.__setattr__(self, "num_aicore_programs", cus)
        object.__setattr__(self, "num_aivector_programs", cus)

        for name in (
            "dispatch_fc1_block_size_m",
            "fc1_gemm_block_size_m",
            "fc1_gemm_block_size_n",
            "fc1_gemm_block_size_k",
            "fc2_combine_block_size_m",
            "fc2_gemm_block_size_n",
            "fc2_gemm_block_size_k",
        ):
            value = getattr(self, name)
            if type(value) is not int or value < 16 or value & (value - 1):
                raise ValueError(f"{name} must be a power of two no smaller than 16")

        single_dispatch_m = self.single_kernel_dispatch_block_size_m
        if single_dispatch_m is None:
            object.__setattr__(self, "single_kernel_dispatch_block_size_m", self.dispatch_fc1_block_size_m)
        elif single_dispatch_m < 16 or single_dispatch_m & (single_dispatch_m - 1):
            raise ValueError(
                "single_kernel_dispatch_block_size_m must be None or a power of two no smaller than 16"
            )

        if self.receive_capacity_factor is not None and self.receive_capacity_factor < 1.0:
            raise ValueError("receive_capacity_factor must be at least 1")
        if self.activation not in _ACTIVATIONS:
            raise ValueError("activation must be one of " + ", ".join(repr(v) for v in _ACTIVATIONS))
        if not (type(self.situ_beta) is float or type(self.situ_beta) is int):
            raise TypeError("situ_beta must be a float")
        if float(self.situ_beta) <= 0.0:
            raise ValueError("situ_beta must be positive")
        if self.situ_linear_beta is not None:
            if not (type(self.situ_linear_beta) is float or type(self.situ_linear_beta) is int):
                raise TypeError("situ_linear_beta must be a float or None")
            if float(self.situ_linear_beta) <= 0.0:
                raise ValueError("situ_linear_beta must be positive when set")
        if not (type(self.clamp_limit) is float or type(self.clamp_limit) is int):
            raise TypeError("clamp_limit must be a float")
        if float(self.clamp_limit) <= 0.0:
            raise ValueError("clamp_limit must be positive")
        if type(self.enable_moonep) is not bool:
            raise TypeError("enable_moonep must be a bool")
        if type(self.enable_single_kernel_forward) is not bool:
            raise TypeError("enable_single_kernel_forward must be a bool")
        if self.save_fc1_dtype not in ("bf16", "fp8", "fp16"):
            raise ValueError('save_fc1_dtype must be "bf16", "fp8" or "fp16"')
        windows = self.single_kernel_group_windows
        if windows is not None and (
            type(windows) is not int or not 1 <= windows <= 64 or windows & (windows - 1)
        ):
            raise ValueError("single_kernel_group_windows must be None or a power of two in [1, 64]")
        if windows is None:
            object.__setattr__(self, "single_kernel_group_windows", 32)
        if self.enable_single_kernel_forward and self.fc1_gemm_block_size_m != self.fc2_combine_block_size_m:
            raise ValueError("single-kernel forward requires matching FC1 and FC2 M tiles")
        for name in ("moonep_fused_balanced_count", "moonep_fused_route_mapping", "moonep_enable_replica_cache"):
            if type(getattr(self, name)) is not bool:
                raise TypeError(f"{name} must be a bool")
        if self.moonep_fused_route_mapping and not self.moonep_fused_balanced_count:
            raise ValueError("moonep_fused_route_mapping requires the fused balanced count cube")

    def resolved_receive_capacity_factor(self, world_size: int) -> float:
        """Return the configured capacity, or the worst-case-safe default."""
        if self.receive_capacity_factor is None:
            return float(world_size)
        return float(self.receive_capacity_factor)


__all__ = ["MoEForwardConfig"]
