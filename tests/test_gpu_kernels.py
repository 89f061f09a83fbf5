"""Parity of each HIP entry point against the CPU oracle / fp32 torch (GPU)."""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from tests._numeric import assert_rel

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _route_gpu(sel, E, rw=None):
    from mega_moe.ops import _kernels as K
    from mega_moe.runtime.routing import route
    from mega_moe import _lib
    need = int(_lib.load().mm_route_workspace_bytes(sel.numel(), E))
    ws = K.workspace(sel.device, need, "route")
    t = route(sel, E, rw, ws)
    torch.cuda.synchronize()
    return t


ROUTE_CASES = [
    # (T, k, E, pattern)
    (0, 2, 8, "uniform"),
    (1, 1, 1, "uniform"),
    (512, 2, 8, "uniform"),
    (333, 3, 7, "drops"),
    (1000, 4, 64, "hot"),
    (4096, 8, 32, "uniform"),
    (4096, 16, 896, "uniform"),
    (8192, 8, 128, "drops"),
    (16384, 8, 32, "zipf"),
    (2049, 5, 1024, "drops"),
    # above 1024 experts: the one-wavefront scatter
    (2049, 5, 1025, "drops"),
    (4096, 8, 4096, "hot"),
    (3000, 16, 20000, "drops"),
    (700, 3, 32768, "uniform"),
]


def _make_sel(T, k, E, pattern, seed):
    rng = np.random.default_rng(seed)
    if pattern == "hot":
        sel = np.zeros((T, k), np.int32)
        sel[:, 1:] = rng.integers(0, E, size=(T, k - 1))
    elif pattern == "zipf":
        p = (np.arange(E) + 1.0) ** -1.2
        p /= p.sum()
        sel = np.stack([rng.choice(E, size=k, replace=False, p=p) for _ in range(T)]).astype(np.int32) \
            if T else np.zeros((0, k), np.int32)
    else:
        sel = rng.integers(0, E, size=(T, k)).astype(np.int32)
    if pattern == "drops" and T:
        m = rng.random((T, k)) < 0.2
        sel[m] = rng.choice([-1, E, E + 7, -100], size=int(m.sum()))
    return sel


@pytest.mark.parametrize("T,k,E,pattern", ROUTE_CASES)
def test_route_bit_exact(T, k, E, pattern):
    sel_np = _make_sel(T, k, E, pattern, seed=T + E)
    sel = torch.from_numpy(sel_np).to(DEV)
    rw = torch.rand(T, k, device=DEV)
    t = _route_gpu(sel, E, rw)
    ref = O.route(sel_np, E, k)
    nv = int(ref["offsets"][-1])
    assert t.offsets.cpu().numpy().tolist() == ref["offsets"].tolist()
    assert t.counts.cpu().numpy().tolist() == ref["counts"].tolist()
    assert np.array_equal(t.send_route[:nv].cpu().numpy(), ref["send_route"])
    assert np.array_equal(t.send_token[:nv].cpu().numpy(), ref["send_token"])
    assert np.array_equal(t.route_to_send.cpu().numpy(), ref["route_to_send"])
    wp = rw.reshape(-1)[torch.from_numpy(ref["send_route"]).long().to(DEV)]
    assert torch.equal(t.weight_perm[:nv], wp)


def _ragged(E, counts_kind, seed, total=None):
    rng = np.random.default_rng(seed)
    if counts_kind == "balanced":
        c = np.full(E, 100)
    elif counts_kind == "ragged":
        c = rng.integers(0, 300, size=E)
        c[0] = 0
        c[-1] = 1
    else:  # skew
        c = (2000 / (np.arange(E) + 1) ** 1.2).astype(int)
    offs = np.zeros(E + 1, np.int32)
    offs[1:] = np.cumsum(c)
    return torch.from_numpy(offs).to(DEV)


def _ref_rows_gemm(a, a_rows, bmat, offs):
    """fp32 reference: c[i] = a[row(i)] @ bmat[e] with bmat[e] [K, N]."""
    offs = offs.cpu().tolist()
    af = a.float().cpu()
    if a_rows is not None:
        af = af[a_rows.long().cpu()]
    out = torch.zeros(offs[-1], bmat.shape[2])
    for e in range(len(offs) - 1):
        if offs[e + 1] > offs[e]:
            out[offs[e]:offs[e + 1]] = af[offs[e]:offs[e + 1]] @ bmat[e].float().cpu()
    return out


@pytest.mark.parametrize("layout", ["kcontig", "ncontig"])
@pytest.mark.parametrize("kind", ["balanced", "ragged", "skew"])
@pytest.mark.parametrize("gather", [False, True])
def test_grouped_gemm(layout, kind, gather):
    from mega_moe.ops import _kernels as K
    E, N, Kd = 6, 256, 192
    offs = _ragged(E, kind, seed=3)
    M = int(offs[-1])
    g = torch.Generator(device=DEV).manual_seed(0)
    src_rows = M + 17
    a = torch.randn(src_rows, Kd, device=DEV, generator=g).to(torch.bfloat16)
    a_rows = torch.randint(0, src_rows, (M,), device=DEV, dtype=torch.int32, generator=g) if gather else None
    if not gather:
        a = a[:M]
    if layout == "kcontig":
        bt = torch.randn(E, N, Kd, device=DEV, generator=g).to(torch.bfloat16)  # B_e(k, n) = bt[e, n, k]
        c = K.grouped_gemm(a, a_rows, bt, bt.stride(0), bt.stride(1), bt.stride(2), offs, M, N, Kd)
        bmat = bt.transpose(1, 2)
    else:
        bm = torch.randn(E, Kd, N, device=DEV, generator=g).to(torch.bfloat16)  # B_e(k, n) = bm[e, k, n]
        c = K.grouped_gemm(a, a_rows, bm, bm.stride(0), bm.stride(2), bm.stride(1), offs, M, N, Kd)
        bmat = bm
    torch.cuda.synchronize()
    ref = _ref_rows_gemm(a, a_rows, bmat, offs)
    assert_rel(c[:M], ref, 1e-2, "grouped_gemm")


@pytest.mark.parametrize("layout", ["kcontig", "ncontig"])
@pytest.mark.parametrize("gather", [False, True])
def test_grouped_gemm_ragged_tails(layout, gather):
    """256-row register-staged tiles (K >= 1024) with every kind of ragged
    last tile: more or fewer than 128 rows, a single row, exact multiples of
    the tile and empty experts."""
    from mega_moe.ops import _kernels as K
    counts = [518, 326, 129, 128, 65, 64, 1, 0, 300, 512, 256, 70]
    E, N, Kd = len(counts), 512, 1024
    offs = torch.tensor([0] + list(np.cumsum(counts)), dtype=torch.int32, device=DEV)
    M = int(offs[-1])
    g = torch.Generator(device=DEV).manual_seed(5)
    src_rows = M + 11
    a = torch.randn(src_rows, Kd, device=DEV, generator=g).to(torch.bfloat16)
    a_rows = torch.randperm(src_rows, device=DEV, generator=g)[:M].to(torch.int32) if gather else None
    if not gather:
        a = a[:M]
    if layout == "kcontig":
        bt = torch.randn(E, N, Kd, device=DEV, generator=g).to(torch.bfloat16)
        c = K.grouped_gemm(a, a_rows, bt, bt.stride(0), bt.stride(1), bt.stride(2), offs, M, N, Kd)
        bmat = bt.transpose(1, 2)
    else:
        bm = torch.randn(E, Kd, N, device=DEV, generator=g).to(torch.bfloat16)
        c = K.grouped_gemm(a, a_rows, bm, bm.stride(0), bm.stride(2), bm.stride(1), offs, M, N, Kd)
        bmat = bm
    torch.cuda.synchronize()
    ref = _ref_rows_gemm(a, a_rows, bmat, offs)
    assert_rel(c[:M], ref, 1e-2, "grouped_gemm")


@pytest.mark.parametrize("layout", ["kcontig", "ncontig"])
@pytest.mark.parametrize("E,N", [(13, 512), (37, 256)])
def test_weight_streaming_xcd_mapping(layout, E, N, monkeypatch):
    """128-row tiles (experts averaging under 96 rows) run M tile m on XCD
    m % 8; with a tile count that is no multiple of 8 (surplus workgroups
    exit) the result is bit-identical to the contiguous per-XCD split
    (MM_XCD_MOD=0) and matches the fp32 reference."""
    from mega_moe.ops import _kernels as K
    g0 = torch.Generator().manual_seed(E)
    counts = torch.randint(0, 140, (E,), generator=g0).tolist()
    offs = torch.tensor([0] + list(np.cumsum(counts)), dtype=torch.int32, device=DEV)
    M, Kd = int(offs[-1]), 320
    g = torch.Generator(device=DEV).manual_seed(7)
    a = torch.randn(M + 5, Kd, device=DEV, generator=g).to(torch.bfloat16)
    a_rows = torch.randperm(M + 5, device=DEV, generator=g)[:M].to(torch.int32)
    if layout == "kcontig":
        b = torch.randn(E, N, Kd, device=DEV, generator=g).to(torch.bfloat16)
        args = (b, b.stride(0), b.stride(1), b.stride(2))
        bmat = b.transpose(1, 2)
    else:
        b = torch.randn(E, Kd, N, device=DEV, generator=g).to(torch.bfloat16)
        args = (b, b.stride(0), b.stride(2), b.stride(1))
        bmat = b
    out = {}
    for mode in ("1", "0"):
        monkeypatch.setenv("MM_XCD_MOD", mode)
        out[mode] = K.grouped_gemm(a, a_rows, *args, offs, M, N, Kd)
    torch.cuda.synchronize()
    assert torch.equal(out["1"][:M], out["0"][:M])
    assert_rel(out["1"][:M], _ref_rows_gemm(a, a_rows, bmat, offs), 1e-2, "grouped_gemm")


@pytest.mark.parametrize("fmt", ["bf16", "fp8"])
def test_fc1_ragged_tails(fmt):
    """FC1 + gated epilogue (and the FP8 save) on the 256-row register-staged
    tiles with every kind of ragged last tile, against a torch fp32
    reference of gate / up and the weighted activation."""
    from mega_moe.ops import _kernels as K
    counts = [518, 326, 129, 128, 65, 64, 1, 0, 300, 70]
    E, H, I = len(counts), 1024, 256
    offs = torch.tensor([0] + list(np.cumsum(counts)), dtype=torch.int32, device=DEV)
    M = int(offs[-1])
    g = torch.Generator(device=DEV).manual_seed(6)
    T = M // 3 + 1
    x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16)
    send_token = torch.randint(0, T, (M,), device=DEV, dtype=torch.int32, generator=g)
    w1 = (torch.randn(E, H, 2 * I, device=DEV, generator=g) * 0.05).to(torch.bfloat16)
    wperm = torch.rand(M, device=DEV, generator=g)
    act, fc1, scale = K.fc1_swiglu(x, send_token, w1, offs, wperm, M, "swiglu", 1.0, None, 7.0, save_fc1=True,
                                   fc1_dtype=fmt)
    torch.cuda.synchronize()
    xp = x.float().cpu()[send_token.long().cpu()]
    o = offs.cpu().tolist()
    gu = torch.zeros(M, 2 * I)
    for e in range(E):
        if o[e + 1] > o[e]:
            gu[o[e]:o[e + 1]] = xp[o[e]:o[e + 1]] @ w1[e].float().cpu()
    gu = gu.to(torch.bfloat16).float()
    ref_act = torch.nn.functional.silu(gu[:, :I]) * gu[:, I:] * wperm.cpu()[:, None]
    assert_rel(act[:M], ref_act, 2e-2, "act")
    if fmt == "bf16":
        assert_rel(fc1[:M], gu, 1e-2, "fc1_output")
    else:
        deq = (fc1[:M].float().cpu().reshape(M, -1, 128) * scale[:M].cpu()[..., None]).reshape(M, 2 * I)
        assert_rel(deq, gu, 7e-2, "fc1_output fp8")


@pytest.mark.parametrize("kind", ["balanced", "ragged", "skew"])
@pytest.mark.parametrize("gather", [False, True])
@pytest.mark.parametrize("tiling", ["wide", "tile", "large", "large_reg"])
def test_grouped_wgrad(kind, gather, tiling, monkeypatch):
    from mega_moe.ops import _kernels as K
    # the kernel variant; read on every call ("large_reg": the register-staged deep-K kernel)
    monkeypatch.setenv("MM_WGRAD_KERNEL", tiling.split("_")[0])
    monkeypatch.setenv("MM_WGRAD_REG", "1" if tiling == "large_reg" else "0")
    E, N1, N2 = 5, 256, 256
    offs = _ragged(E, kind, seed=4)
    M = int(offs[-1])
    g = torch.Generator(device=DEV).manual_seed(1)
    p = torch.randn(M + 9, N1, device=DEV, generator=g).to(torch.bfloat16)
    q = torch.randn(M, N2, device=DEV, generator=g).to(torch.bfloat16)
    p_rows = torch.randint(0, M + 9, (M,), device=DEV, dtype=torch.int32, generator=g) if gather else None
    c = K.grouped_wgrad(p, p_rows, q, None, offs, N1, N2, max_rows=M)
    torch.cuda.synchronize()
    pf = p.float().cpu()
    pf = pf[p_rows.long().cpu()] if gather else pf[:M]
    qf = q.float().cpu()
    o = offs.cpu().tolist()
    ref = torch.zeros(E, N1, N2)
    for e in range(E):
        ref[e] = pf[o[e]:o[e + 1]].T @ qf[o[e]:o[e + 1]]
    assert_rel(c, ref, 1e-2, "grouped_wgrad")
    for e in range(E):
        if o[e + 1] == o[e]:
            assert torch.count_nonzero(c[e]) == 0


@pytest.mark.parametrize("shape", [(512, 1280), (1280, 512)], ids=["n2_tiles_more", "n1_tiles_more"])
@pytest.mark.parametrize("tiling", ["wide", "tile", "large_reg"])
def test_grouped_wgrad_many_experts_both_gathered(tiling, shape, monkeypatch):
    """Small-K regime with many experts: rows 0..140 per expert (zero-row
    experts, a last K stage of <= 16 rows, multi-stage K, one 300-row
    expert), both operands gathered (read in place)."""
    from mega_moe.ops import _kernels as K
    monkeypatch.setenv("MM_WGRAD_KERNEL", tiling.split("_")[0])
    monkeypatch.setenv("MM_WGRAD_REG", "1" if tiling == "large_reg" else "0")
    E = 21
    N1, N2 = shape  # both tile walks of the small-K kernel (more tiles along n1 or along n2)
    rng = np.random.default_rng(11)
    cnt = rng.integers(0, 141, size=E)
    cnt[[2, 9]] = 0
    cnt[5] = 300
    offs = torch.from_numpy(np.concatenate([[0], np.cumsum(cnt)]).astype(np.int32)).to(DEV)
    M = int(offs[-1])
    g = torch.Generator(device=DEV).manual_seed(2)
    p = torch.randn(M + 3, N1, device=DEV, generator=g).to(torch.bfloat16)
    q = torch.randn(M + 5, N2, device=DEV, generator=g).to(torch.bfloat16)
    p_rows = torch.randint(0, M + 3, (M,), device=DEV, dtype=torch.int32, generator=g)
    q_rows = torch.randperm(M + 5, device=DEV, generator=g)[:M].to(torch.int32)
    c = K.grouped_wgrad(p, p_rows, q, q_rows, offs, N1, N2, max_rows=M)
    torch.cuda.synchronize()
    pf = p.float().cpu()[p_rows.long().cpu()]
    qf = q.float().cpu()[q_rows.long().cpu()]
    o = offs.cpu().tolist()
    ref = torch.zeros(E, N1, N2)
    for e in range(E):
        ref[e] = pf[o[e]:o[e + 1]].T @ qf[o[e]:o[e + 1]]
    assert_rel(c, ref, 1e-2, "grouped_wgrad")
    assert torch.count_nonzero(c[2]) == 0 and torch.count_nonzero(c[9]) == 0


def test_combine_integer_exact():
    from mega_moe.ops import _kernels as K
    T, k, H = 300, 6, 384
    rows = T * k
    y = (torch.arange(rows * H, device=DEV) % 23 - 11).to(torch.bfloat16).view(rows, H)
    perm = torch.randperm(rows, device=DEV).to(torch.int32)
    perm[::7] = -1
    out = K.combine(y, perm, T, k)
    torch.cuda.synchronize()
    yf = y.float().cpu()
    p = perm.view(T, k).long().cpu()
    ref = torch.zeros(T, H)
    for j in range(k):
        m = p[:, j] >= 0
        ref[m] += yf[p[m, j]]
    assert torch.equal(out.float().cpu(), ref)


def test_permute_exact():
    from mega_moe.ops import _kernels as K
    x = torch.randn(100, 256, device=DEV).to(torch.bfloat16)
    st = torch.randint(0, 100, (400,), device=DEV, dtype=torch.int32)
    offs = torch.tensor([0, 150, 150, 390], dtype=torch.int32, device=DEV)
    out = K.permute(x, st, offs, 400)
    torch.cuda.synchronize()
    assert torch.equal(out[:390], x[st[:390].long()])


@pytest.mark.parametrize("activation", ["swiglu", "clamp_swiglu", "situglu"])
@pytest.mark.parametrize("fmt", ["bf16", "fp16", "fp8"])
def test_swiglu_bwd(activation, fmt):
    from mega_moe.ops import _kernels as K
    M, inter = 300, 256
    g = torch.Generator(device=DEV).manual_seed(5)
    fc1 = torch.randn(M, 2 * inter, device=DEV, generator=g).to(torch.bfloat16)
    ga = torch.randn(M, inter, device=DEV, generator=g).to(torch.bfloat16)
    sc = torch.rand(M, device=DEV, generator=g)
    offs = torch.tensor([0, 100, 290], dtype=torch.int32, device=DEV)
    kw = dict(activation=activation, situ_beta=1.5, situ_linear_beta=2.0 if activation == "situglu" else None,
              clamp_limit=0.5)
    q, qs = O.quantize_fc1(fc1.float().cpu(), fmt)   # saved form of the FC1 values in this format
    dab, ds = K.swiglu_bwd(ga, q.to(DEV), sc, offs, M, fc1_scale=None if qs is None else qs.to(DEV), **kw)
    torch.cuda.synchronize()
    fcd = O.dequantize_fc1(q, qs)
    gate, up = fcd[:290, :inter], fcd[:290, inter:]
    act_a, dact, v, dv = O.gated_act_grad(gate, up, **kw)
    s = O.bf16(sc[:290].cpu())[:, None]
    gaf = ga[:290].float().cpu()
    ref_dab = torch.cat([gaf * dact * v * s, gaf * act_a * dv * s], 1)
    ref_ds = (act_a * v * gaf).sum(1)
    assert_rel(dab[:290], ref_dab, 1e-2, "dab")
    assert_rel(ds[:290], ref_ds, 1e-2, "dscale")


@pytest.mark.parametrize("T,k,H", [(300, 6, 384), (129, 16, 7168), (1, 1, 128)])
def test_combine_bwd_one_launch(T, k, H):
    """mm_combine_bwd = mm_combine + mm_gather_route_grad in one launch: the
    top-k reduce exact on integer rows, grad_rw gathered from dscale with 0
    for dropped routes, both equal to the two-launch results."""
    from mega_moe.ops import _kernels as K
    rows = T * k
    y = (torch.arange(rows * H, device=DEV) % 23 - 11).to(torch.bfloat16).view(rows, H)
    perm = torch.randperm(rows, device=DEV).to(torch.int32)
    perm[::7] = -1
    dscale = torch.randn(rows, device=DEV).to(torch.bfloat16)
    gh, grw = K.combine_bwd(y, perm, T, k, dscale)
    ref_h = K.combine(y, perm, T, k)
    ref_rw = K.gather_route_grad(dscale, perm, (T, k))
    torch.cuda.synchronize()
    assert torch.equal(gh, ref_h) and torch.equal(grw, ref_rw)
    p = perm.view(T, k).long()
    want = torch.where(p >= 0, dscale.float()[p.clamp(min=0)], torch.zeros_like(grw))
    assert torch.equal(grw, want)
