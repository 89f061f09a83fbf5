"""CPU oracle of the Mega-MoE layer -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker or the timed CPU baseline. The
product path (mega_moe) never calls it.

A restatement, written for this repository, of the reference's algorithm:

* routing     runtime/routing.py:621-671 (valid mask, float32 *stable*
              argsort by expert id, token = route // k, histogram, exclusive
              offsets) and kernels/fc2_combine.py:508-529 (inverse, -1 for
              dropped routes) -- numpy, integer exact.
* forward     tests/_moe_baselines.py:326-471 (torch_moe_fwd_golden) at one
              rank: per-expert fp32 GEMMs of bf16 operands, gate and up
              rounded to bf16, act = bf16(act_fn(gate, up) * w) with w in
              fp32, FC2 rounded to bf16, combine = fp32 sum over the k slots in
              slot order, rounded to bf16. The gated activation variants follow
              ops/_torch_forward.py:177-205.
* saved FC1   save_fc1_dtype bf16 / fp16 / fp8 (E4M3 + per-row, per-128-
              column fp32 scales) per kernels/fused_forward.py:888-937, read
              back per kernels/mega_bwd.py:264-270.
* backward    tests/_moe_baselines.py:96-226 (moe_backward_torch) at one
              rank, swiglu_bwd per tests/_moe_baselines.py:122-160 and
              kernels/swiglu_bwd.py:52-83 (scale = the bf16-cast routing
              weight, as the reference's saved recv_weights_sorted), every
              GEMM output rounded to bf16 as the reference's bf16 matmuls are.
* sampled     backward_tokens / backward_expert: the same forward and
              backward formulas restricted to chosen tokens (output,
              grad_hidden, grad_routing_weights rows) or to one expert's
              weight gradients, so full-size configurations can be checked
              on the CPU.

Where each function is pinned (tests/test_oracle.py): routing against a
pure-Python brute-force stable sort plus the reference's invariants
(tests/function/test_single_kernel_stable_scatter.py); the forward against a
per-token fp64 dense evaluation; combine with integer-valued rows (exact);
the backward against torch.autograd of an fp64 restatement of the forward
(as src/mega_moe/_goldens/backward.py:200-283 cross-checks it); the FP8
quantizer against the closed-form E4M3 value of every code (round trip,
ties-to-even at every midpoint, saturation) and its per-group invariants
(max |q| = 448, error <= half an E4M3 step); backward_tokens and
backward_expert bit for bit against the full backward (all tokens, every
expert, bf16 and narrowed FC1 saves).
"""

from __future__ import annotations

import numpy as np
import torch

ACTIVATIONS = ("swiglu", "situglu", "clamp_swiglu")


def bf16(t: torch.Tensor) -> torch.Tensor:
    """Round to bf16 (RNE) and return as fp32."""
    return t.to(torch.bfloat16).to(torch.float32)


def _mm(a: torch.Tensor, b: torch.Tensor, dtype=torch.float32) -> torch.Tensor:
    """a @ b with operands in ``dtype`` (fp32: the checker; bf16: bf16 GEMMs
    with fp32 accumulation, as the reference's Torch path runs them), fp32
    result."""
    return (a.to(dtype) @ b.to(dtype)).float()


# --------------------------------------------------------------------- routing
def route(selected: np.ndarray, num_experts: int, top_k: int) -> dict:
    """Stable expert-major routing tables (runtime/routing.py:621-671)."""
    flat = np.asarray(selected, dtype=np.int64).reshape(-1)
    valid = (flat >= 0) & (flat < num_experts)
    kept = np.nonzero(valid)[0]
    order = np.argsort(flat[kept].astype(np.float32), kind="stable")
    send_route = kept[order].astype(np.int32)
    counts = np.bincount(flat[kept], minlength=num_experts).astype(np.int32)
    offsets = np.zeros(num_experts + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    route_to_send = np.full(flat.shape[0], -1, dtype=np.int32)
    route_to_send[send_route] = np.arange(send_route.shape[0], dtype=np.int32)
    return dict(
        send_route=send_route,
        send_token=(send_route // top_k).astype(np.int32),
        counts=counts,
        offsets=offsets,
        route_to_send=route_to_send,
        stable_sort_indices=order.astype(np.int64),
        valid=valid,
    )


# --------------------------------------------------------------------- activation
def gated_act(g, u, activation="swiglu", situ_beta=1.0, situ_linear_beta=None, clamp_limit=7.0):
    """act(gate) * v(up) in the input precision (ops/_torch_forward.py:177-205)."""
    if activation == "swiglu":
        return torch.nn.functional.silu(g) * u
    if activation == "clamp_swiglu":
        return torch.nn.functional.silu(g.clamp(max=clamp_limit)) * u.clamp(min=-clamp_limit, max=clamp_limit)
    if activation == "situglu":
        a = situ_beta * torch.tanh(g / situ_beta) * torch.sigmoid(g)
        if situ_linear_beta is not None:
            u = situ_linear_beta * torch.tanh(u / situ_linear_beta)
        return a * u
    raise ValueError(activation)


def gated_act_grad(g, u, activation="swiglu", situ_beta=1.0, situ_linear_beta=None, clamp_limit=7.0):
    """(act_a, dact_a, v, dv) per tests/_moe_baselines.py:122-160 and kernels/swiglu_bwd.py:52-83."""
    if activation == "swiglu":
        s = torch.sigmoid(g)
        act_a = g * s
        return act_a, act_a * (1 - s) + s, u, torch.ones_like(u)
    if activation == "clamp_swiglu":
        L = clamp_limit
        gc = g.clamp(max=L)
        s = torch.sigmoid(gc)
        act_a = gc * s
        dact = (s + gc * s * (1 - s)) * (g <= L).to(g.dtype)
        return act_a, dact, u.clamp(min=-L, max=L), (u.abs() <= L).to(u.dtype)
    t = torch.tanh(g / situ_beta)
    s = torch.sigmoid(g)
    act_a = situ_beta * t * s
    dact = (1 - t * t) * s + situ_beta * t * s * (1 - s)
    if situ_linear_beta is not None:
        tu = torch.tanh(u / situ_linear_beta)
        return act_a, dact, situ_linear_beta * tu, 1 - tu * tu
    return act_a, dact, u, torch.ones_like(u)


# --------------------------------------------------------------------- saved FC1 formats
FP8_MAX = 448.0          # largest finite E4M3 ("fn") value
FC1_SCALE_GROUP = 128    # columns per FP8 scale (fc1_gemm_block_size_n // 2 at its default 256)


def e4m3fn_value(code: int) -> float:
    """Closed-form value of an 8-bit E4M3 "fn" code (bias 7, no infinities,
    0x7F / 0xFF = NaN): the definition the quantizer below is pinned to."""
    sign = -1.0 if code & 0x80 else 1.0
    e, m = (code >> 3) & 0xF, code & 7
    if e == 15 and m == 7:
        return float("nan")
    if e == 0:
        return sign * m * 2.0 ** -9
    return sign * (1.0 + m / 8.0) * 2.0 ** (e - 7)


def quantize_fc1(gu: torch.Tensor, fmt: str):
    """Saved form of the raw FC1 output gu [M, 2I] (bf16 values held in fp32).

    bf16 / fp16: the values cast (kernels/fused_forward.py:888-901).
    fp8: per row and per 128-column group (gate groups, then up groups),
    amax = max |value| (1 for an all-zero group), q = E4M3(value * (448 /
    amax)) rounded to nearest even and saturated at 448, scale = amax / 448
    (kernels/fused_forward.py:902-937). Returns (stored, scale | None).
    """
    if fmt == "bf16":
        return gu.to(torch.bfloat16), None
    if fmt == "fp16":
        return gu.to(torch.float16), None
    if fmt != "fp8":
        raise ValueError(fmt)
    M, two_i = gu.shape
    g = gu.float().reshape(M, two_i // FC1_SCALE_GROUP, FC1_SCALE_GROUP)
    amax = g.abs().amax(dim=2)
    safe = torch.where(amax > 0, amax, torch.ones_like(amax))
    # correctly rounded fp32 division (a python-scalar / tensor expression
    # would be evaluated as scalar * reciprocal(tensor), one more rounding)
    mult = torch.full_like(safe, FP8_MAX) / safe
    q = (g * mult[..., None]).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q.reshape(M, two_i), safe / FP8_MAX


def dequantize_fc1(stored: torch.Tensor, scale=None) -> torch.Tensor:
    """fp32 values of a saved FC1 output (value = e4m3 * scale for fp8;
    kernels/mega_bwd.py:264-270)."""
    if stored.dtype == torch.float8_e4m3fn:
        M, two_i = stored.shape
        return (stored.float().reshape(M, -1, FC1_SCALE_GROUP) * scale[..., None]).reshape(M, two_i)
    return stored.float()


# --------------------------------------------------------------------- forward
def forward(x, selected, gate_up, down, rw, activation="swiglu", situ_beta=1.0, situ_linear_beta=None,
            clamp_limit=7.0, save_fc1_dtype="bf16", matmul_dtype=torch.float32):
    """Layer forward on CPU.

    ``matmul_dtype`` bf16 runs the GEMMs on bf16 operands (the timed CPU
    baseline); every GEMM output is rounded to bf16 either way.

    x [T, H] bf16; selected [T, k] int32; gate_up [E, H, 2I] bf16;
    down [E, H, I] bf16 (any strides); rw [T, k] fp32.
    Returns (out [T, H] bf16, state dict for ``backward``).
    """
    T, H = x.shape
    k = selected.shape[1]
    E, _, two_i = gate_up.shape
    inter = two_i // 2
    tb = route(selected.cpu().numpy(), E, k)
    send_token = torch.from_numpy(tb["send_token"]).long()
    send_route = torch.from_numpy(tb["send_route"]).long()
    offsets = tb["offsets"]
    xf = x.float().cpu()
    mm = matmul_dtype
    w1 = gate_up.cpu().to(mm)
    w2 = down.cpu().to(mm)
    wp = rw.float().cpu().reshape(-1)[send_route]
    M = send_route.numel()
    gate = torch.empty(M, inter)
    up = torch.empty(M, inter)
    y = torch.empty(M, H)
    xp = xf[send_token]
    for e in range(E):
        a, b = int(offsets[e]), int(offsets[e + 1])
        if a == b:
            continue
        gu = _mm(xp[a:b], w1[e], mm)
        gate[a:b] = bf16(gu[:, :inter])
        up[a:b] = bf16(gu[:, inter:])
    act = bf16(gated_act(gate, up, activation, situ_beta, situ_linear_beta, clamp_limit) * wp[:, None])
    for e in range(E):
        a, b = int(offsets[e]), int(offsets[e + 1])
        if a == b:
            continue
        y[a:b] = bf16(_mm(act[a:b], w2[e].T, mm))
    r2s = torch.from_numpy(tb["route_to_send"]).long().view(T, k)
    out = torch.zeros(T, H)
    for j in range(k):
        rows = r2s[:, j]
        m = rows >= 0
        out[m] += y[rows[m]]
    fc1_saved, fc1_scale = quantize_fc1(torch.cat([gate, up], dim=1), save_fc1_dtype)
    state = dict(tables=tb, x=xf, w1=w1, w2=w2, wp=wp, gate=gate, up=up, act=act, y=y, T=T, k=k, E=E,
                 inter=inter, activation=activation, situ_beta=situ_beta, situ_linear_beta=situ_linear_beta,
                 clamp_limit=clamp_limit, fc1_output=fc1_saved, fc1_output_scale=fc1_scale, mm=mm)
    return out.to(torch.bfloat16), state


def forward_tokens(x, selected, gate_up, down, rw, tokens, activation="swiglu", situ_beta=1.0,
                   situ_linear_beta=None, clamp_limit=7.0):
    """Forward output rows for a subset of tokens only (same rounding points).

    Lets a test check full-size configurations on sampled tokens.
    """
    E, H, two_i = gate_up.shape
    inter = two_i // 2
    k = selected.shape[1]
    rows = []
    for t in tokens:
        acc = torch.zeros(H)
        xt = x[t].float().cpu()
        for j in range(k):
            e = int(selected[t, j])
            if not 0 <= e < E:
                continue
            gu = xt @ gate_up[e].float().cpu()
            g, u = bf16(gu[:inter]), bf16(gu[inter:])
            a = bf16(gated_act(g, u, activation, situ_beta, situ_linear_beta, clamp_limit) * float(rw[t, j]))
            acc += bf16(down[e].float().cpu() @ a)
        rows.append(acc.to(torch.bfloat16))
    return torch.stack(rows)


# --------------------------------------------------------------------- backward
def backward(state, dy, recompute_act=False):
    """Five-stage backward on CPU (tests/_moe_baselines.py:96-226).

    ``recompute_act``: the FC2 weight gradient reads the weighted activation
    recomputed from the saved (maybe narrowed) FC1 output, as the reference's
    MOE_SAVED_RECOMPUTE mode does (kernels/mega_bwd.py:1414-1468).
    """
    tb = state["tables"]
    T, k, E, inter = state["T"], state["k"], state["E"], state["inter"]
    offsets = tb["offsets"]
    send_token = torch.from_numpy(tb["send_token"]).long()
    w1, w2 = state["w1"], state["w2"]
    mm = state.get("mm", torch.float32)
    dyf = dy.float().cpu()
    H = dyf.shape[1]
    gco = bf16(dyf)[send_token]                                   # step 1a
    M = gco.shape[0]
    grad_act = torch.empty(M, inter)
    for e in range(E):                                            # step 1b
        a, b = int(offsets[e]), int(offsets[e + 1])
        if a < b:
            grad_act[a:b] = bf16(_mm(gco[a:b], w2[e], mm))
    scale = bf16(state["wp"])[:, None]                            # step 2
    gu = dequantize_fc1(state["fc1_output"], state.get("fc1_output_scale"))  # the saved (maybe narrowed) FC1
    act_a, dact, v, dv = gated_act_grad(gu[:, :inter], gu[:, inter:], state["activation"], state["situ_beta"],
                                        state["situ_linear_beta"], state["clamp_limit"])
    dgate = grad_act * dact * v * scale
    dup = grad_act * act_a * dv * scale
    dab = bf16(torch.cat([dgate, dup], dim=1))
    dscale = bf16((act_a * v * grad_act).sum(dim=1))
    act_saved = state["act"]
    if recompute_act:
        act_saved = bf16(gated_act(gu[:, :inter], gu[:, inter:], state["activation"], state["situ_beta"],
                                   state["situ_linear_beta"], state["clamp_limit"]) * state["wp"][:, None])
    grad_fc2 = torch.zeros(E, H, inter)                           # step 3
    dx = torch.empty(M, H)
    grad_gate_up = torch.zeros(E, H, 2 * inter)
    xp = state["x"][send_token]
    for e in range(E):
        a, b = int(offsets[e]), int(offsets[e + 1])
        if a == b:
            continue
        grad_fc2[e] = bf16(_mm(gco[a:b].T, act_saved[a:b], mm))
        dx[a:b] = bf16(_mm(dab[a:b], w1[e].T, mm))                      # step 4a
        grad_gate_up[e] = bf16(_mm(xp[a:b].T, dab[a:b], mm))            # step 5
    r2s = torch.from_numpy(tb["route_to_send"]).long().view(T, k)
    grad_hidden = torch.zeros(T, H)                               # step 4b
    grad_rw = torch.zeros(T, k)
    for j in range(k):
        rows = r2s[:, j]
        m = rows >= 0
        grad_hidden[m] += dx[rows[m]]
        grad_rw[m, j] = dscale[rows[m]]
    return dict(
        grad_hidden=grad_hidden.to(torch.bfloat16),
        grad_routing_weights=grad_rw,
        grad_fc2=grad_fc2.to(torch.bfloat16),
        grad_gate_up=grad_gate_up.to(torch.bfloat16),
        grad_swiglu=grad_act,
        grad_fc1_output=dab,
        grad_gate=dscale,
        grad_fc2_out_sorted=gco,
        grad_recv_hidden_sorted=dx,
    )


# --------------------------------------------------------------------- sampled backward
def _expert_rows(xr, dyr, wr, w1e, w2e, activation, situ_beta, situ_linear_beta, clamp_limit, save_fc1_dtype="bf16"):
    """Forward and backward quantities of one expert's rows (same rounding
    points as ``forward`` / ``backward``).

    xr, dyr [n, H] fp32 (bf16 values); wr [n] fp32 routing weights;
    w1e [H, 2I], w2e [H, I] fp32. Every GEMM here has the operand shapes the
    per-expert loops of ``forward`` / ``backward`` use for the same rows, so
    for an expert's complete row set the results are bit-identical to theirs.
    """
    inter = w1e.shape[1] // 2
    gu = xr @ w1e
    gate, up = bf16(gu[:, :inter]), bf16(gu[:, inter:])
    act = bf16(gated_act(gate, up, activation, situ_beta, situ_linear_beta, clamp_limit) * wr[:, None])
    y = bf16(act @ w2e.T)
    gco = bf16(dyr)
    grad_act = bf16(gco @ w2e)                                        # step 1
    scale = bf16(wr)[:, None]                                         # step 2
    # the backward reads the saved (maybe narrowed) FC1 output, as ``backward`` does
    saved, sc = quantize_fc1(torch.cat([gate, up], dim=1), save_fc1_dtype)
    gu = dequantize_fc1(saved, sc)
    act_a, dact, v, dv = gated_act_grad(gu[:, :inter], gu[:, inter:], activation, situ_beta, situ_linear_beta,
                                        clamp_limit)
    dab = bf16(torch.cat([grad_act * dact * v * scale, grad_act * act_a * dv * scale], dim=1))
    dscale = bf16((act_a * v * grad_act).sum(dim=1))
    dx = bf16(dab @ w1e.T)                                            # step 4a
    return dict(act=act, y=y, gco=gco, dab=dab, dscale=dscale, dx=dx)


def _act_kw(kw):
    return (kw.get("activation", "swiglu"), kw.get("situ_beta", 1.0), kw.get("situ_linear_beta"),
            kw.get("clamp_limit", 7.0), kw.get("save_fc1_dtype", "bf16"))


def backward_tokens(x, selected, gate_up, down, rw, dy, tokens, **act_kw):
    """Layer output and input gradients for a subset of tokens only.

    Restates forward steps FC1 -> act -> FC2 -> combine and backward steps
    1, 2 and 4 (tests/_moe_baselines.py:96-226: gco gather, FC2 dgrad,
    gated-activation backward, FC1 dgrad, top-k reduce in slot order,
    grad_routing_weights = dscale of the route's row, 0 if dropped) for the
    routes of ``tokens``; the routes of one expert are evaluated together, so
    each expert's weights are read once. Inputs may live on any device; the
    arithmetic runs on the CPU in fp32 with bf16 rounding. ``act_kw`` takes
    the activation arguments of ``forward`` and ``save_fc1_dtype`` (the
    backward reads the saved FC1 output in that format, as ``backward`` does).

    Returns dict(out [n, H] bf16, grad_hidden [n, H] bf16,
    grad_routing_weights [n, k] fp32) in the order of ``tokens``.
    """
    kw = _act_kw(act_kw)
    tokens = [int(t) for t in tokens]
    E, H, two_i = gate_up.shape
    sel = selected.cpu().long()
    k = sel.shape[1]
    by_expert: dict = {}
    for n, t in enumerate(tokens):
        for j in range(k):
            e = int(sel[t, j])
            if 0 <= e < E:
                by_expert.setdefault(e, []).append((n, j))
    xs = x[tokens].float().cpu()
    dys = dy[tokens].float().cpu()
    ws = rw[tokens].float().cpu()
    y_rows, dx_rows = {}, {}
    grad_rw = torch.zeros(len(tokens), k)
    for e in sorted(by_expert):
        nj = by_expert[e]
        idx = torch.tensor([n for n, _ in nj])
        slot = torch.tensor([j for _, j in nj])
        r = _expert_rows(xs[idx], dys[idx], ws[idx, slot], gate_up[e].cpu().float(), down[e].cpu().float(), *kw)
        for i, (n, j) in enumerate(nj):
            y_rows[n, j] = r["y"][i]
            dx_rows[n, j] = r["dx"][i]
            grad_rw[n, j] = r["dscale"][i]
    out = torch.zeros(len(tokens), H)
    grad_hidden = torch.zeros(len(tokens), H)
    for n in range(len(tokens)):
        for j in range(k):                     # fp32 sum in slot order
            if (n, j) in y_rows:
                out[n] += y_rows[n, j]
                grad_hidden[n] += dx_rows[n, j]
    return dict(out=out.to(torch.bfloat16), grad_hidden=grad_hidden.to(torch.bfloat16), grad_routing_weights=grad_rw)


def backward_expert(x, selected, gate_up, down, rw, dy, expert, **act_kw):
    """Weight gradients of one expert (backward steps 3 and 5 of
    tests/_moe_baselines.py:96-226): grad_fc2[e] = bf16(gco_e^T act_e) [H, I]
    and grad_gate_up[e] = bf16(x_e^T dAB_e) [H, 2I], over the expert's rows in
    the stable expert-major order (ascending flat route id). Inputs may live
    on any device; returns (grad_gate_up_e, grad_fc2_e) bf16 on the CPU.
    """
    kw = _act_kw(act_kw)
    E, H, two_i = gate_up.shape
    e = int(expert)
    flat = selected.cpu().long().reshape(-1)
    routes = torch.nonzero(flat == e).reshape(-1)            # ascending = stable order
    k = selected.shape[1]
    if routes.numel() == 0:
        z = torch.zeros
        return z(H, two_i, dtype=torch.bfloat16), z(H, two_i // 2, dtype=torch.bfloat16)
    toks = routes // k
    dev_toks = toks.to(x.device)
    xr = x.index_select(0, dev_toks).float().cpu()
    dyr = dy.index_select(0, dev_toks).float().cpu()
    wr = rw.reshape(-1).index_select(0, routes.to(rw.device)).float().cpu()
    r = _expert_rows(xr, dyr, wr, gate_up[e].cpu().float(), down[e].cpu().float(), *kw)
    return bf16(xr.T @ r["dab"]).to(torch.bfloat16), bf16(r["gco"].T @ r["act"]).to(torch.bfloat16)


# --------------------------------------------------------------------- fp64 autograd restatement
def reference_autograd(x, selected, gate_up, down, rw, dy, activation="swiglu", situ_beta=1.0,
                       situ_linear_beta=None, clamp_limit=7.0):
    """Dense per-token fp64 forward + torch.autograd gradients (no rounding).

    Independent of ``route``: each token loops over its own k slots. Used to
    pin ``forward`` and ``backward`` against the calculus, not against
    themselves. The only rounding kept is gate/up -> bf16 (value only), so the
    piecewise clamp derivative is taken on the same side as in the oracle.
    """
    xd = x.double().cpu().clone().requires_grad_(True)
    rwd = rw.double().cpu().clone().requires_grad_(True)
    w1 = gate_up.double().cpu().clone().requires_grad_(True)
    w2 = down.double().cpu().clone().requires_grad_(True)
    T, k = selected.shape
    E, H, two_i = gate_up.shape
    inter = two_i // 2
    outs = []
    for t in range(T):
        acc = torch.zeros(H, dtype=torch.float64)
        for j in range(k):
            e = int(selected[t, j])
            if not 0 <= e < E:
                continue
            gu = xd[t] @ w1[e]
            # evaluate act and its derivative at the bf16-rounded gate/up, as
            # the reference does (straight-through: value rounded, gradient 1)
            gu = gu + (gu.to(torch.bfloat16).double() - gu).detach()
            a = gated_act(gu[:inter], gu[inter:], activation, situ_beta, situ_linear_beta, clamp_limit) * rwd[t, j]
            acc = acc + w2[e] @ a
        outs.append(acc)
    out = torch.stack(outs)
    out.backward(dy.double().cpu())
    return dict(out=out.detach(), grad_hidden=xd.grad, grad_routing_weights=rwd.grad, grad_gate_up=w1.grad,
                grad_fc2=w2.grad)
