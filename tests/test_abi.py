"""The C-ABI library loads and exports every symbol include/megamoe.h declares
(no compute calls: runs without a GPU)."""

import ctypes
import os
import re

import pytest

from mega_moe import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "megamoe.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mm_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for s in ("mm_route", "mm_fc1_swiglu", "mm_grouped_gemm", "mm_grouped_wgrad", "mm_combine", "mm_swiglu_bwd",
              "mm_permute", "mm_gather_route_grad", "mm_last_error"):
        assert s in syms


@pytest.mark.skipif(not os.path.exists(_lib.library_path()), reason="libmegamoe.so not built")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.library_path())
    for s in declared_symbols():
        assert hasattr(lib, s), f"libmegamoe.so does not export {s}"
        assert s in _lib.SIGNATURES, f"python binding lacks a prototype for {s}"


@pytest.mark.skipif(not os.path.exists(_lib.library_path()), reason="libmegamoe.so not built")
def test_host_side_argument_errors():
    # Argument validation runs on the host and never touches a device.
    lib = _lib.load()
    rc = lib.mm_route(None, 10, 2, 0, None, None, None, None, None, None, None, None, 0, None)
    assert rc == -1 and b"num_experts" in lib.mm_last_error()
    rc = lib.mm_grouped_gemm(None, 0, None, None, 0, 0, 0, None, 1, 1, 100, 64, None, 0, None, 0, None)
    assert rc == -1
    assert lib.mm_route_workspace_bytes(131072, 896) >= 64 * 896 * 4


@pytest.mark.skipif(not os.path.exists(_lib.library_path()), reason="libmegamoe.so not built")
def test_wgrad_needs_no_workspace():
    """Every weight-gradient kernel gathers its rows in place, so
    mm_wgrad_workspace_bytes (kept for the ABI) reports 0 at every size."""
    lib = _lib.load()
    E, n1, n2 = 896, 7168, 4096
    assert [lib.mm_wgrad_workspace_bytes(r, E, n1, n2) for r in (0, 1, 4096 * 16, 16384 * 16)] == [0, 0, 0, 0]

@pytest.mark.skipif(not os.path.exists(_lib.library_path()), reason="libmegamoe.so not built")
def test_wgrad_rejects_row_strides_past_32_bits():
    """The weight-gradient kernels form row addresses with one 32 x 32-bit
    multiply, so the host rejects row strides of 2^32 elements or more (the
    check runs before any device call; the pointers are never read)."""
    lib = _lib.load()
    fake = ctypes.c_void_p(1 << 20)  # 16-byte aligned, never dereferenced
    args = lambda ldp, ldq: (fake, ldp, None, fake, ldq, None, fake, 8, 1024, 256, 256, fake, None, 0, None)
    rc = lib.mm_grouped_wgrad(*args(1 << 32, 256))
    assert rc == -1 and b"2^32" in lib.mm_last_error()
    rc = lib.mm_grouped_wgrad(*args(256, (1 << 32) + 8))
    assert rc == -1 and b"2^32" in lib.mm_last_error()


@pytest.mark.skipif(not os.path.exists(_lib.library_path()), reason="libmegamoe.so not built")
def test_grouped_gemm_rejects_grids_past_32_bits():
    """A row GEMM whose largest tile grid would not fit a 32-bit launch size is
    rejected on the host before any launch (the pointers are never read)."""
    lib = _lib.load()
    fake = ctypes.c_void_p(1 << 20)
    max_rows, E, n, k = (1 << 31) - 1, 8, 65536, 64
    rc = lib.mm_grouped_gemm(fake, k, None, fake, n * k, 1, n, fake, E, max_rows, n, k, fake, n, fake, 1 << 40, None)
    assert rc == -1 and b"too many tiles" in lib.mm_last_error()
