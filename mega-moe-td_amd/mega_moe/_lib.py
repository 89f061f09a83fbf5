"""ctypes binding of libmegamoe.so, the C ABI declared in include/megamoe.h.

The shared library is built in-tree (``__graft_entry__.build()`` or
``make -C mega-moe-td_amd/csrc``). There is no fallback: if the library is
missing every device entry point raises, so a GPU run can never silently
execute a CPU or PyTorch substitute.
"""

from __future__ import annotations

import ctypes
import os

import torch

_LIB_PATH = os.environ.get("MEGAMOE_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmegamoe.so")

# Activation kinds (include/megamoe.h MM_ACT_*).
ACT_KINDS = {"swiglu": 0, "situglu": 1, "clamp_swiglu": 2}
# saved FC1 output formats (MM_FC1_* in include/megamoe.h) and the FP8 scale group
FC1_FORMATS = {"bf16": 0, "fp16": 1, "fp8": 2}
FC1_SCALE_GROUP = 128

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t
_F32 = ctypes.c_float

# name -> (restype, argtypes); mirrors include/megamoe.h one to one.
SIGNATURES = {
    "mm_last_error": (ctypes.c_char_p, []),
    "mm_version": (ctypes.c_int, []),
    "mm_route_workspace_bytes": (_SZ, [_I64, _I32]),
    "mm_route": (ctypes.c_int, [_P, _I64, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "mm_route_noalloc_scratch_bytes": (_SZ, []),
    "mm_route_noalloc": (ctypes.c_int, [_P, _I64, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P]),
    "mm_permute": (ctypes.c_int, [_P, _I64, _P, _P, _I32, _I64, _I32, _P, _I64, _P]),
    "mm_gemm_workspace_bytes": (_SZ, [_I64, _I32]),
    "mm_wgrad_workspace_bytes": (_SZ, [_I64, _I32, _I32, _I32]),
    "mm_fc1_swiglu": (ctypes.c_int, [_P, _I64, _P, _P, _P, _P, _I32, _I64, _I32, _I32, _I32,
                                     _F32, _F32, _F32, _P, _P, _I32, _P, _P, _SZ, _P]),
    "mm_grouped_gemm": (ctypes.c_int, [_P, _I64, _P, _P, _I64, _I64, _I64, _P, _I32, _I64, _I32,
                                       _I32, _P, _I64, _P, _SZ, _P]),
    "mm_grouped_wgrad": (ctypes.c_int, [_P, _I64, _P, _P, _I64, _P, _P, _I32, _I64, _I32, _I32, _P, _P,
                                        _SZ, _P]),
    "mm_combine": (ctypes.c_int, [_P, _I64, _P, _I64, _I32, _I32, _P, _I64, _P]),
    "mm_gather_route_grad": (ctypes.c_int, [_P, _P, _I64, _P, _P]),
    "mm_combine_bwd": (ctypes.c_int, [_P, _I64, _P, _I64, _I32, _I32, _P, _I64, _P, _P, _P]),
    "mm_gated_act": (ctypes.c_int, [_P, _I64, _I32, _P, _P, _P, _I32, _I64, _I32, _I32, _F32, _F32, _F32, _P,
                                    _I64, _P]),
    "mm_swiglu_bwd": (ctypes.c_int, [_P, _I64, _P, _I64, _I32, _P, _P, _P, _I32, _I64, _I32, _I32, _F32,
                                     _F32, _F32, _P, _P, _P]),
}

_lib = None


def library_path() -> str:
    return _LIB_PATH


def load() -> ctypes.CDLL:
    """Load libmegamoe.so (once) and attach the C prototypes."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        raise RuntimeError(
            f"libmegamoe.so not found at {_LIB_PATH}; build it with "
            "`python -c 'import __graft_entry__ as g; g.build()'` or "
            "`make -C mega-moe-td_amd/csrc`")
    lib = ctypes.CDLL(_LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


class MegaMoEError(RuntimeError):
    """A libmegamoe entry point rejected its arguments or failed to launch."""


def call(name: str, *args):
    """Call a status-returning entry point and raise on a non-zero status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.mm_last_error().decode(errors="replace")
        raise MegaMoEError(f"{name} failed ({rc}): {msg}")


def ptr(t: torch.Tensor | None):
    """Raw device address of a tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(device: torch.device):
    """Handle of torch's current HIP stream on `device`."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
