"""Five-stage MoE backward on one MI355X.

Mirrors ``moe_backward_triton`` (src/mega_moe/ops/backward.py:100-399) and the
hand-written reference backward it is checked against
(tests/_moe_baselines.py:96-226). Given dy [T, H]:

  1. FC2 dgrad   grad_act = gco @ down[e]      gco = dy[send_token] is gathered
                                              inside the GEMM's A-tile load
  2. SwiGLU bwd  dAB = [dGate | dUp], dscale   (mm_swiglu_bwd)
  3. FC2 wgrad   dW2[e] = gco_e^T act_e        (mm_grouped_wgrad, rows gathered)
  4. FC1 dgrad   dX = dAB @ W1[e]^T, then grad_hidden = top-k sum of dX and
                 grad_routing_weights = dscale gathered to [T, k]
  5. FC1 wgrad   dW1[e] = X_e^T dAB_e          (X rows re-gathered from
                 hidden_states, written directly in the packed [E, H, 2I]
                 gate_up layout)

Returned keys follow the reference: grad_hidden, grad_routing_weights,
grad_fc1_1 / grad_fc1_2 ([E, F, H] views), grad_fc2 ([E, H, F]) and the
intermediates grad_swiglu, grad_fc1_output, grad_gate, grad_fc1 (plus
grad_fc2_out_sorted, derived when read, and grad_recv_hidden_sorted when
``saved["_keep_grad_recv_hidden_sorted"]`` is set); plus grad_gate_up, the
packed [E, H, 2F] weight gradient.
"""

from __future__ import annotations

import torch

import os

from ..runtime.timing import NULL_TIMER, StageTimer
from . import _kernels as K
from .forward import saved_recompute


# Step 2 (the gated-activation backward, HBM-bound) runs on a second stream
# beside step 3 (the FC2 weight gradient) when experts average more than
# _OVERLAP_ROWS route-capacity rows: there the deep-K weight gradient is
# MFMA-bound and the activation backward fills idle HBM bandwidth. Whole-layer
# A/B in one process (interleaved groups of steps), overlap off -> on:
# Skew-like 14.553 -> 14.507 and 14.409 -> 14.382 ms per step; Qwen-like
# (512 rows) 2.632 -> 2.637 and 2.594 -> 2.618; Kimi-scale (73 rows, both
# kernels HBM-bound) 41.16 -> 41.16 and 41.00 -> 41.52.
_OVERLAP_ROWS = 1024
_SIDE_STREAMS: dict = {}


def overlap_act_bwd(num_routes: int, num_experts: int) -> bool:
    """Whether step 2 runs on a second stream beside step 3: by default for
    experts averaging more than ``_OVERLAP_ROWS`` route-capacity rows;
    ``MM_BWD_ACT_OVERLAP=0`` / ``=1`` forces it off / on."""
    env = os.environ.get("MM_BWD_ACT_OVERLAP")
    if env in ("0", "1"):
        return env == "1"
    return num_routes > _OVERLAP_ROWS * num_experts


def _side_stream(device) -> torch.cuda.Stream:
    key = str(device)
    st = _SIDE_STREAMS.get(key)
    if st is None:
        st = torch.cuda.Stream(device=device)  # default priority
        _SIDE_STREAMS[key] = st
    return st


def moe_backward_triton(saved, dy, peer_mem=None, grad_transport=None, hidden_states=None):
    """Run the five backward stages on a ``saved`` dict from ``FusedMoEForward``.

    ``peer_mem`` is accepted for signature compatibility (one GPU has no
    symmetric buffer); ``grad_transport`` (MoonEP) must be ``None``.
    """
    if grad_transport is not None:
        raise NotImplementedError("MoonEP replica gradient transport is not built")
    if saved.get("batch_size") == 0:
        return _empty_batch_grads(saved, dy)
    if "fc1_output" not in saved:
        raise ValueError("saved is missing fc1_output; run the forward with return_saved=True")
    T = saved["batch_size"]
    k = saved["topk"]
    H = saved["hidden_dim"]
    inter = saved["ffn_dim"]
    R = saved["total_routes"]
    w1 = saved["gate_up_weight"]
    w2 = saved["down_weight"]
    offsets = saved["split_size_cum_per_expert"]
    send_token = saved["send_token_indices"]
    r2s = saved["route_to_send"]
    x = hidden_states if hidden_states is not None else saved["hidden_states"]
    if dy.shape != (T, H):
        raise ValueError(f"dy must have shape {(T, H)}, got {tuple(dy.shape)}")
    if x.shape != (T, H) or x.dtype != torch.bfloat16 or not x.is_contiguous():
        raise ValueError(f"hidden_states must be a contiguous bf16 tensor of shape {(T, H)}")
    dy = dy.to(torch.bfloat16).contiguous()
    act_kw = dict(activation=saved["activation"], situ_beta=saved["situ_beta"],
                  situ_linear_beta=saved["situ_linear_beta"], clamp_limit=saved["clamp_limit"])

    tm = saved.get("_stage_timer") or NULL_TIMER
    # MOE_BWD_STAGE_TIMING=1 (reference ops/backward.py:216-230, 333-347): HIP
    # events around the stages of this pass, summed into the reference's five
    # intervals and appended to saved["_bwd_stage_samples"]
    stage_timing = os.environ.get("MOE_BWD_STAGE_TIMING") == "1"
    if stage_timing and tm is NULL_TIMER:
        tm = StageTimer()
    tm.mark_pass()
    pool = saved.get("_workspaces")
    ws_rows = saved.get("_max_routes") or R
    # step 1: FC2 dgrad, B_e(k=h, n=f) = down[e, h, f]
    tm.begin("fc2_dgrad")
    se, sh, sf = w2.stride()
    grad_act = K.grouped_gemm(dy, send_token, w2, se, sf, sh, offsets, R, inter, H, pool=pool)
    tm.end()
    # step 2: gated-activation backward
    side = _side_stream(dy.device) if overlap_act_bwd(R, offsets.numel() - 1) else None
    if side is None:  # overlapped with step 3 otherwise: its time is part of "fc2_wgrad"
        tm.begin("swiglu_bwd")
    fc1_scale = None
    if saved["fc1_output"].dtype == torch.float8_e4m3fn:
        # FP8 save: dequantize at the load (reference kernels/mega_bwd.py:3185-3206)
        fc1_scale = saved.get("fc1_output_scale")
        if fc1_scale is None or int(saved.get("fc1_scale_group_size", 0)) != 128:
            raise ValueError("an FP8 fc1_output needs fc1_output_scale with fc1_scale_group_size 128")
    if side is None:
        dab, dscale = K.swiglu_bwd(grad_act, saved["fc1_output"], saved["recv_weights_sorted"], offsets, R,
                                   fc1_scale=fc1_scale, **act_kw)
    else:
        # step 2 (HBM-bound, no LDS) on a second stream beside step 3 (the
        # MFMA-bound deep-K weight gradient): its waves fit in the register
        # and LDS space the GEMM's one workgroup per CU leaves free (the
        # reference's step 2 || step 3, ops/backward.py:241-271)
        # The outputs come from the main stream's pool and are not recorded
        # on the side stream (the main stream waits for it before any use or
        # release): allocated on the side stream, or recorded there, dAB
        # moved between steps and the FC1 dgrad that reads it ran 0.3-0.7 ms
        # slower at Kimi scale (same kernel and data, one process).
        main = torch.cuda.current_stream(dy.device)
        dab = torch.empty(R, 2 * inter, dtype=torch.bfloat16, device=dy.device)
        dscale = torch.empty(R, dtype=torch.bfloat16, device=dy.device)
        side.wait_stream(main)
        with torch.cuda.stream(side):
            K.swiglu_bwd(grad_act, saved["fc1_output"], saved["recv_weights_sorted"], offsets, R,
                         fc1_scale=fc1_scale, out=(dab, dscale), **act_kw)
        for t in (grad_act, saved["fc1_output"], saved["recv_weights_sorted"], offsets, fc1_scale):
            if t is not None:
                t.record_stream(side)
    if side is None:
        tm.end()
    # step 3: FC2 wgrad  dW2[e][h, f] = sum_i gco[i, h] act[i, f]
    act = saved.get("swiglu_out_weighted")
    if act is None or saved_recompute():
        # MOE_SAVED_RECOMPUTE: act from the saved FC1 output (reference kernels/mega_bwd.py:1414-1468)
        tm.begin("act_recompute")
        act = K.gated_act(saved["fc1_output"], saved["recv_weights_sorted"], offsets, R, fc1_scale=fc1_scale,
                          **act_kw)
        tm.end()
    tm.begin("fc2_wgrad")
    grad_fc2 = K.grouped_wgrad(dy, send_token, act, None, offsets, H, inter, pool=pool, ws_rows=ws_rows)
    if side is not None:
        main.wait_stream(side)
    tm.end()
    # step 4: FC1 dgrad, B_e(k=j, n=h) = W1[e, h, j]; top-k reduce; gate gather
    tm.begin("fc1_dgrad")
    dx = K.grouped_gemm(dab, None, w1, w1.stride(0), w1.stride(1), 1, offsets, R, H, 2 * inter, pool=pool)
    tm.end()
    tm.begin("combine_bwd")
    grad_hidden, grad_rw = K.combine_bwd(dx, r2s, T, k, dscale)
    tm.end()
    # step 5: FC1 wgrad in the packed layout  dW1[e][h, j] = sum_i x[tok(i), h] dAB[i, j]
    tm.begin("fc1_wgrad")
    grad_gate_up = K.grouped_wgrad(x, send_token, dab, None, offsets, H, 2 * inter, pool=pool, ws_rows=ws_rows)
    tm.end()

    grads = _grad_dict(grad_hidden, grad_rw, grad_fc2, grad_gate_up, grad_act, dab, dscale, inter)
    # dx [R, H] is released here unless the caller asked to keep the
    # pre-reduction FC1 input gradient (a per-stage check, not a training need)
    grads._bind(dy, send_token, offsets, dx if saved.get("_keep_grad_recv_hidden_sorted") else None)
    if stage_timing:
        _record_stage_sample(saved, tm, act_overlapped=side is not None)
    return grads


# The reference's five backward intervals and the stages of this build that
# make them up (its combine_fc1_bwd holds the FC1 dgrad and the top-k reduce).
_BWD_INTERVALS = (
    ("dispatch", ("fc2_dgrad",)),
    ("fc2_wgrad", ("act_recompute", "fc2_wgrad")),
    ("swiglu", ("swiglu_bwd",)),
    ("fc1_wgrad", ("fc1_wgrad",)),
    ("combine", ("fc1_dgrad", "combine_bwd")),
)


def _record_stage_sample(saved, timer, act_overlapped=False):
    """Append this pass's [dispatch, fc2_wgrad, swiglu, fc1_wgrad, combine]
    milliseconds to saved["_bwd_stage_samples"] and print them (synchronises).
    With the activation backward on the second stream its time is inside
    fc2_wgrad and the swiglu interval is NaN (not measured on its own)."""
    last = timer.last_pass()
    sample = [sum(last.get(s, 0.0) for s in stages) for _, stages in _BWD_INTERVALS]
    if act_overlapped:
        sample[[n for n, _ in _BWD_INTERVALS].index("swiglu")] = float("nan")
    saved.setdefault("_bwd_stage_samples", []).append(sample)
    print("[bwd-stage] " + " ".join(f"{v:8.3f}" for v in sample), flush=True)


class MoEGrads(dict):
    """Gradient dict of ``moe_backward_triton``.

    Besides the gradients it derives, on first read, the two expert-major
    intermediates the reference exposes for per-stage checks
    (tests/_moe_baselines.py:208-225, ops/backward.py:384-399):
    ``grad_fc2_out_sorted`` = dy gathered to the expert-major rows [M, H]
    (the backward's GEMMs read it in place, so it is materialised only when
    asked for) and ``grad_recv_hidden_sorted`` = the FC1 input gradient
    [M, H] before the top-k reduce, kept only when the saved dict sets
    ``_keep_grad_recv_hidden_sorted`` (it holds R x H bf16 otherwise freed
    after the reduce). M = number of valid routes (one host read of the
    routing offsets).
    """

    _DERIVED = ("grad_fc2_out_sorted", "grad_recv_hidden_sorted")

    def _bind(self, dy, send_token, offsets, dx):
        self._src = (dy, send_token, offsets, dx)

    def __missing__(self, key):
        if not self._has_derived(key):
            raise KeyError(key)
        dy, send_token, offsets, dx = self._src
        m = int(offsets[-1].item())
        if key == "grad_fc2_out_sorted":
            value = K.permute(dy, send_token, offsets, m) if m else dy[:0].clone()
        else:
            value = dx[:m]
        self[key] = value
        return value

    def _has_derived(self, key):
        src = getattr(self, "_src", None)
        if key not in self._DERIVED or src is None:
            return False
        return key != "grad_recv_hidden_sorted" or src[3] is not None

    def __contains__(self, key):
        return dict.__contains__(self, key) or self._has_derived(key)

    def get(self, key, default=None):
        try:
            return self[key]
        except KeyError:
            return default


def _grad_dict(grad_hidden, grad_rw, grad_fc2, grad_gate_up, grad_act, dab, dscale, inter):
    grad_fc1 = grad_gate_up.transpose(1, 2)  # [E, 2F, H] view
    return MoEGrads(
        grad_hidden=grad_hidden,
        grad_routing_weights=grad_rw,
        grad_fc1_1=grad_fc1[:, :inter],
        grad_fc1_2=grad_fc1[:, inter:],
        grad_fc2=grad_fc2,
        grad_gate_up=grad_gate_up,
        grad_swiglu=grad_act,
        grad_fc1_output=dab,
        grad_gate=dscale,
        grad_fc1=grad_fc1,
    )


def _empty_batch_grads(saved, dy):
    """Gradients of a zero-token batch: empty input gradients and all-zero
    weight gradients (no expert received a row)."""
    H, inter, k = saved["hidden_dim"], saved["ffn_dim"], saved["topk"]
    if tuple(dy.shape) != (0, H):
        raise ValueError(f"dy must have shape {(0, H)}, got {tuple(dy.shape)}")
    w1 = saved["gate_up_weight"]
    dev, bf = w1.device, torch.bfloat16
    E = w1.shape[0]
    grads = _grad_dict(torch.empty(0, H, dtype=bf, device=dev), torch.empty(0, k, dtype=torch.float32, device=dev),
                       torch.zeros(E, H, inter, dtype=bf, device=dev), torch.zeros(E, H, 2 * inter, dtype=bf, device=dev),
                       torch.empty(0, inter, dtype=bf, device=dev), torch.empty(0, 2 * inter, dtype=bf, device=dev),
                       torch.empty(0, dtype=bf, device=dev), inter)
    grads.update(grad_fc2_out_sorted=torch.empty(0, H, dtype=bf, device=dev),
                 grad_recv_hidden_sorted=torch.empty(0, H, dtype=bf, device=dev))
    return grads


class MegaMoEBackwardFunction(torch.autograd.Function):
    """Autograd function over unpacked weights (reference ops/backward.py:405-455).

    Arguments: hidden_states [B, H], routing_weights [B, k] fp32,
    selected_experts [B, k] int32, fc1_1 / fc1_2 [E, F, H], fc2 [E, H, F],
    ep_group (None on one GPU), topk, peer_mem (unused placeholder).
    """

    @staticmethod
    def forward(ctx, hidden_states, routing_weights, selected_experts, fc1_1, fc1_2, fc2, ep_group, topk,
                peer_mem):
        from .forward import FusedMoEForward, pack_gate_up_weights

        E, F, H = fc1_1.shape
        op = FusedMoEForward(ep_group, max_tokens_per_rank=max(1, hidden_states.shape[0]), hidden_size=H,
                             top_k=topk, num_experts=E)
        gate_up = pack_gate_up_weights(fc1_1, fc1_2)
        with torch.no_grad():
            output, saved = op.forward(hidden_states.contiguous(), selected_experts.contiguous(), gate_up, fc2,
                                       routing_weights.contiguous(), return_saved=True)
        ctx.saved = saved
        ctx.inter = F
        return output

    @staticmethod
    def backward(ctx, dy):
        grads = moe_backward_triton(ctx.saved, dy)
        return (grads["grad_hidden"], grads["grad_routing_weights"], None, grads["grad_fc1_1"],
                grads["grad_fc1_2"], grads["grad_fc2"], None, None, None)


__all__ = ["MegaMoEBackwardFunction", "MoEGrads", "moe_backward_triton"]
