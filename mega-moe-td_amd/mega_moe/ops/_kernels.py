"""Thin torch-facing wrappers over the libmegamoe C ABI.

Each function allocates its outputs with torch (the C ABI itself never
allocates), launches one entry point on the current stream, and returns the
outputs. Shapes are checked here before any launch so a kernel never sees a
grid or operand it does not expect.
"""

from __future__ import annotations

import torch

from .. import _lib

class WorkspacePool:
    """Byte workspaces per (device, stream, tag) that never move under a
    captured graph.

    Calls on one stream are ordered, so they share a workspace; work on
    another stream gets its own, so concurrent streams never race on a tile
    list. A workspace that a larger call outgrows is retired, not freed: a
    HIP graph captured earlier keeps its address baked in, and the retired
    buffer stays valid for that graph's replays until ``release()``.
    ``FusedMoEForward`` owns one pool sized for its ``max_tokens_per_rank`` at
    the first forward, so its own calls never grow it; the module pool serves
    direct calls of these wrappers and grows by powers of two
    (``geometric``), so a caller with steadily growing sizes retires at most
    one buffer per doubling per (device, stream, tag).
    """

    def __init__(self, geometric: bool = False):
        self._live: dict = {}
        self._retired: list = []
        self._geometric = geometric

    def get(self, device: torch.device, nbytes: int, tag: str) -> torch.Tensor:
        key = (str(device), torch.cuda.current_stream(device).cuda_stream, tag)
        ws = self._live.get(key)
        if ws is None or ws.numel() < nbytes:
            if ws is not None:
                self._retired.append(ws)
            size = max(nbytes, 256)
            if self._geometric:
                size = 1 << (size - 1).bit_length()
            ws = torch.empty(size, dtype=torch.uint8, device=device)
            self._live[key] = ws
        return ws

    def nbytes(self) -> int:
        return sum(t.numel() for t in self._live.values()) + sum(t.numel() for t in self._retired)

    def release(self):
        """Drop every workspace (no graph captured over them may replay after this)."""
        self._live.clear()
        self._retired.clear()


_POOL = WorkspacePool(geometric=True)


def workspace(device: torch.device, nbytes: int, tag: str, pool: WorkspacePool | None = None) -> torch.Tensor:
    return (pool or _POOL).get(device, nbytes, tag)


def gemm_workspace_bytes(max_rows: int, num_experts: int) -> int:
    return int(_lib.load().mm_gemm_workspace_bytes(max_rows, num_experts))


def route_workspace_bytes(num_routes: int, num_experts: int) -> int:
    return int(_lib.load().mm_route_workspace_bytes(num_routes, num_experts))


def wgrad_workspace_bytes(max_rows: int, num_experts: int, n1: int, n2: int) -> int:
    return int(_lib.load().mm_wgrad_workspace_bytes(max_rows, num_experts, n1, n2))


def _gemm_ws(device, max_rows: int, num_experts: int, pool=None) -> torch.Tensor:
    return workspace(device, gemm_workspace_bytes(max_rows, num_experts), "gemm", pool)


def _check_bf16(name: str, t: torch.Tensor):
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be torch.bfloat16, got {t.dtype}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a HIP device tensor")


def permute(x: torch.Tensor, send_token: torch.Tensor, offsets: torch.Tensor, max_rows: int) -> torch.Tensor:
    """out[i] = x[send_token[i]] for the valid expert-major rows."""
    _check_bf16("x", x)
    hidden = x.shape[1]
    out = torch.empty(max_rows, hidden, dtype=x.dtype, device=x.device)
    _lib.call("mm_permute", _lib.ptr(x), x.stride(0), _lib.ptr(send_token), _lib.ptr(offsets),
              offsets.numel() - 1, max_rows, hidden, _lib.ptr(out), out.stride(0), _lib.stream_of(x.device))
    return out


_FC1_TORCH_DTYPE = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp8": torch.float8_e4m3fn}


def fc1_format_of(t: torch.Tensor) -> str:
    """Saved-FC1 format name of a tensor's dtype."""
    for name, dt in _FC1_TORCH_DTYPE.items():
        if t.dtype == dt:
            return name
    raise TypeError(f"fc1_output dtype {t.dtype} is not bf16, fp16 or float8_e4m3fn")


def fc1_swiglu(x, send_token, w1, offsets, weight_perm, max_rows: int, activation: str, situ_beta: float,
               situ_linear_beta, clamp_limit: float, save_fc1: bool, fc1_dtype: str = "bf16", pool=None):
    """FC1 grouped GEMM + weighted gated activation.

    Returns (act [rows, I] bf16, fc1_output [rows, 2I] in ``fc1_dtype`` | None,
    fc1_scale [rows, 2I / 128] fp32 for fp8 | None).
    """
    _check_bf16("x", x)
    _check_bf16("w1", w1)
    num_experts, hidden, two_inter = w1.shape
    inter = two_inter // 2
    if x.shape[1] != hidden or not w1.is_contiguous() or x.stride(1) != 1:
        raise ValueError("fc1_swiglu: x [*, H] and contiguous w1 [E, H, 2I] required")
    if fc1_dtype not in _FC1_TORCH_DTYPE:
        raise ValueError(f"fc1_dtype must be one of {sorted(_FC1_TORCH_DTYPE)}, got {fc1_dtype!r}")
    dev = x.device
    act = torch.empty(max_rows, inter, dtype=torch.bfloat16, device=dev)
    fc1_out = torch.empty(max_rows, two_inter, dtype=_FC1_TORCH_DTYPE[fc1_dtype], device=dev) if save_fc1 else None
    fc1_scale = None
    if save_fc1 and fc1_dtype == "fp8":
        if inter % _lib.FC1_SCALE_GROUP:
            raise ValueError(f"fp8 fc1 save needs ffn % {_lib.FC1_SCALE_GROUP} == 0, got {inter}")
        fc1_scale = torch.empty(max_rows, two_inter // _lib.FC1_SCALE_GROUP, dtype=torch.float32, device=dev)
    ws = _gemm_ws(dev, max_rows, num_experts, pool)
    lbeta = float(situ_linear_beta) if situ_linear_beta is not None else 0.0
    _lib.call("mm_fc1_swiglu", _lib.ptr(x), x.stride(0), _lib.ptr(send_token), _lib.ptr(w1), _lib.ptr(offsets),
              _lib.ptr(weight_perm), num_experts, max_rows, hidden, inter, _lib.ACT_KINDS[activation],
              float(situ_beta), lbeta, float(clamp_limit), _lib.ptr(act), _lib.ptr(fc1_out),
              _lib.FC1_FORMATS[fc1_dtype], _lib.ptr(fc1_scale), _lib.ptr(ws), ws.numel(), _lib.stream_of(dev))
    return act, fc1_out, fc1_scale


def grouped_gemm(a, a_rows, b, b_se: int, b_sn: int, b_sk: int, offsets, max_rows: int, n: int, k: int,
                 pool=None):
    """c[i, :] = a[row(i), :] @ B_e for expert-major rows; B_e(k, n) = b[e*se + n*sn + k*sk]."""
    _check_bf16("a", a)
    _check_bf16("b", b)
    if a.stride(1) != 1 or a.shape[1] != k:
        raise ValueError("grouped_gemm: a must be [*, K] with unit column stride")
    num_experts = offsets.numel() - 1
    c = torch.empty(max_rows, n, dtype=torch.bfloat16, device=a.device)
    ws = _gemm_ws(a.device, max_rows, num_experts, pool)
    _lib.call("mm_grouped_gemm", _lib.ptr(a), a.stride(0), _lib.ptr(a_rows), _lib.ptr(b), b_se, b_sn, b_sk,
              _lib.ptr(offsets), num_experts, max_rows, n, k, _lib.ptr(c), c.stride(0), _lib.ptr(ws), ws.numel(),
              _lib.stream_of(a.device))
    return c


def grouped_wgrad(p, p_rows, q, q_rows, offsets, n1: int, n2: int, max_rows: int | None = None, pool=None,
                  ws_rows: int | None = None) -> torch.Tensor:
    """c[e] = P_e^T Q_e over each expert's rows -> [E, n1, n2] bf16.

    Gathered rows (``p_rows`` / ``q_rows``) are read in place; the kernels
    take no workspace (``pool`` and ``ws_rows`` are accepted for the callers
    that pass them)."""
    _check_bf16("p", p)
    _check_bf16("q", q)
    if p.stride(1) != 1 or q.stride(1) != 1 or p.shape[1] != n1 or q.shape[1] != n2:
        raise ValueError("grouped_wgrad: p [*, n1], q [*, n2] with unit column stride required")
    num_experts = offsets.numel() - 1
    if max_rows is None:
        max_rows = q.shape[0] if q_rows is None else q_rows.shape[0]
    c = torch.empty(num_experts, n1, n2, dtype=torch.bfloat16, device=p.device)
    _lib.call("mm_grouped_wgrad", _lib.ptr(p), p.stride(0), _lib.ptr(p_rows), _lib.ptr(q), q.stride(0),
              _lib.ptr(q_rows), _lib.ptr(offsets), num_experts, max_rows, n1, n2, _lib.ptr(c), None, 0,
              _lib.stream_of(p.device))
    return c


def combine(y, route_to_send, num_tokens: int, top_k: int) -> torch.Tensor:
    """out[t] = bf16(sum_j fp32(y[route_to_send[t*k+j]])) (dropped routes skipped)."""
    _check_bf16("y", y)
    hidden = y.shape[1]
    out = torch.empty(num_tokens, hidden, dtype=torch.bfloat16, device=y.device)
    _lib.call("mm_combine", _lib.ptr(y), y.stride(0), _lib.ptr(route_to_send), num_tokens, top_k, hidden,
              _lib.ptr(out), out.stride(0), _lib.stream_of(y.device))
    return out


def combine_bwd(dx, route_to_send, num_tokens: int, top_k: int, dscale):
    """(grad_hidden [T, H] bf16, grad_rw [T, k] fp32) in one launch: the top-k
    reduce of dx and the gather of dscale to the routes (0 where dropped)."""
    _check_bf16("dx", dx)
    hidden = dx.shape[1]
    gh = torch.empty(num_tokens, hidden, dtype=torch.bfloat16, device=dx.device)
    grw = torch.empty(num_tokens, top_k, dtype=torch.float32, device=dx.device)
    _lib.call("mm_combine_bwd", _lib.ptr(dx), dx.stride(0), _lib.ptr(route_to_send), num_tokens, top_k, hidden,
              _lib.ptr(gh), gh.stride(0), _lib.ptr(dscale), _lib.ptr(grw), _lib.stream_of(dx.device))
    return gh, grw


def swiglu_bwd(grad_act, fc1_out, scale, offsets, max_rows: int, activation: str, situ_beta: float,
               situ_linear_beta, clamp_limit: float, fc1_scale=None, out=None):
    """Gated-activation backward -> (dAB [rows, 2I] bf16, dscale [rows] bf16).

    ``fc1_out`` is the saved raw FC1 output in bf16, fp16 or float8_e4m3fn
    (then with its fp32 ``fc1_scale`` [rows, 2I / 128]). ``out`` optionally
    supplies the two result tensors (allocated by the caller).
    """
    _check_bf16("grad_act", grad_act)
    fmt = fc1_format_of(fc1_out)
    if fc1_out.device.type != "cuda" or fc1_out.stride(1) != 1:
        raise ValueError("fc1_out must be a HIP device tensor with unit column stride")
    inter = fc1_out.shape[1] // 2
    if fmt == "fp8":
        if fc1_scale is None or fc1_scale.dtype != torch.float32 or not fc1_scale.is_contiguous() or \
                tuple(fc1_scale.shape) != (fc1_out.shape[0], 2 * inter // _lib.FC1_SCALE_GROUP):
            raise ValueError("fp8 fc1_out needs an fp32 contiguous fc1_scale [rows, 2F // 128]")
    dev = fc1_out.device
    if out is None:
        dab = torch.empty(max_rows, 2 * inter, dtype=torch.bfloat16, device=dev)
        dscale = torch.empty(max_rows, dtype=torch.bfloat16, device=dev)
    else:
        dab, dscale = out
        if dab.dtype != torch.bfloat16 or tuple(dab.shape) != (max_rows, 2 * inter) or not dab.is_contiguous() \
                or dscale.dtype != torch.bfloat16 or tuple(dscale.shape) != (max_rows,) or not dscale.is_contiguous() \
                or dab.device != dev or dscale.device != dev:
            raise ValueError(f"swiglu_bwd out must be contiguous bf16 [{max_rows}, {2 * inter}] and [{max_rows}] "
                             "tensors on the fc1_out device")
    lbeta = float(situ_linear_beta) if situ_linear_beta is not None else 0.0
    _lib.call("mm_swiglu_bwd", _lib.ptr(grad_act), grad_act.stride(0), _lib.ptr(fc1_out), fc1_out.stride(0),
              _lib.FC1_FORMATS[fmt], _lib.ptr(fc1_scale if fmt == "fp8" else None), _lib.ptr(scale),
              _lib.ptr(offsets), offsets.numel() - 1, max_rows, inter, _lib.ACT_KINDS[activation],
              float(situ_beta), lbeta, float(clamp_limit), _lib.ptr(dab), _lib.ptr(dscale), _lib.stream_of(dev))
    return dab, dscale


def gather_route_grad(dscale, route_to_send, shape) -> torch.Tensor:
    """grad_rw[r] = float(dscale[route_to_send[r]]), 0 for dropped routes."""
    out = torch.empty(shape, dtype=torch.float32, device=dscale.device)
    _lib.call("mm_gather_route_grad", _lib.ptr(dscale), _lib.ptr(route_to_send), out.numel(), _lib.ptr(out),
              _lib.stream_of(dscale.device))
    return out


def gated_act(fc1_out, weight_perm, offsets, max_rows: int, activation: str, situ_beta: float, situ_linear_beta,
              clamp_limit: float, fc1_scale=None) -> torch.Tensor:
    """act [rows, I] bf16 recomputed from a saved FC1 output (bf16 / fp16 / fp8 + scale)."""
    fmt = fc1_format_of(fc1_out)
    if fc1_out.device.type != "cuda" or fc1_out.stride(1) != 1:
        raise ValueError("fc1_out must be a HIP device tensor with unit column stride")
    inter = fc1_out.shape[1] // 2
    if fmt == "fp8" and (fc1_scale is None or fc1_scale.dtype != torch.float32 or not fc1_scale.is_contiguous()):
        raise ValueError("fp8 fc1_out needs an fp32 contiguous fc1_scale")
    act = torch.empty(max_rows, inter, dtype=torch.bfloat16, device=fc1_out.device)
    lbeta = float(situ_linear_beta) if situ_linear_beta is not None else 0.0
    _lib.call("mm_gated_act", _lib.ptr(fc1_out), fc1_out.stride(0), _lib.FC1_FORMATS[fmt],
              _lib.ptr(fc1_scale if fmt == "fp8" else None), _lib.ptr(weight_perm), _lib.ptr(offsets),
              offsets.numel() - 1, max_rows, inter, _lib.ACT_KINDS[activation], float(situ_beta), lbeta,
              float(clamp_limit), _lib.ptr(act), act.stride(0), _lib.stream_of(fc1_out.device))
    return act
