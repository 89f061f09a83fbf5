"""FP8-saved FC1 output (GPU): why a large layer's per-expert FC1 weight
gradient can sit just past the 2e-2 bar against the independent oracle while
every kernel is right.

The build and the oracle round FC1 to E4M3 codes (with one fp32 scale per
row and 128-column group) from fp32 sums taken in different orders, so a
value at a rounding tie can take the neighbouring code, and a group amax one
bf16 ulp away moves the group's scale. One E4M3 step is 6-12% of the value,
so such an element of the saved FC1 moves its ``grad_fc1_output`` element,
and that element moves a whole column of the expert's FC1 weight gradient.

A one-off fuzz of large layers found one such case (fuzz case 104, SiTU-GLU,
dW1 of expert 7 2.04e-2 off); this test re-runs it with its fuzz seed and
checks, for the probed experts,
  (i)  the build's saved codes equal the oracle's within one step where the
       group scale agrees, and the scales within one bf16 ulp of the amax,
  (ii) the FC1 weight gradient equals the oracle's backward on the build's
       own save within 2e-2 (the same formula, fed the build's save).
"""

import pytest
import torch

import mega_moe
from mega_moe.bench_configs import CaseSpec, make_inputs
from oracle import moe_oracle as O
from tests._fc1_save import bf16_ulp, e4m3_magnitude_index
from tests._numeric import max_rel
from tests.test_gpu_layer import _act_kw, _op, _probe_experts

pytestmark = pytest.mark.gpu


def test_fp8_save_code_flips_explain_expert_gap():
    i, T, H, I, E, k, routing = 104, 6144, 5120, 1024, 96, 16, "softmax_topk"
    print(f"fp8 save flip case fuzz{i} T{T} H{H} I{I} E{E} top-{k}", flush=True)
    spec = CaseSpec("fuzz", T, H, I, E, k, routing, True)
    inp = make_inputs(spec, device="cuda", seed=100 + i)
    kw = _act_kw("situglu")
    op = _op(spec, "situglu", save_fc1_dtype="fp8", **{a: b for a, b in kw.items() if a != "activation"})
    x, sel, w1, w2, rw, dy = inp["x"], inp["selected"], inp["gate_up"], inp["down"], inp["rw"], inp["dy"]
    out, saved = op.forward(x, sel, w1, w2, rw, return_saved=True)
    g = mega_moe.moe_backward_triton(saved, dy)
    torch.cuda.synchronize()
    ka = O._act_kw(dict(kw, save_fc1_dtype="fp8"))
    offs = saved["split_size_cum_per_expert"].cpu()
    counts = (offs[1:] - offs[:-1]).tolist()
    flat = sel.cpu().long().reshape(-1)
    for e in sorted({7, *_probe_experts(counts)[:2]}):
        a0, a1 = int(offs[e]), int(offs[e + 1])
        routes = torch.nonzero(flat == e).reshape(-1)
        toks = (routes // k).to(x.device)
        xr = x.index_select(0, toks).float().cpu()
        dyr = dy.index_select(0, toks).float().cpu()
        wr = rw.reshape(-1).index_select(0, routes.to(rw.device)).float().cpu()
        w1e, w2e = w1[e].cpu().float(), w2[e].cpu().float()
        own = O._expert_rows(xr, dyr, wr, w1e, w2e, *ka)
        # (i) the two FP8 saves of the expert's rows
        gu = xr @ w1e
        codes_o, sc_o = O.quantize_fc1(torch.cat([O.bf16(gu[:, :I]), O.bf16(gu[:, I:])], dim=1), "fp8")
        codes_b = saved["fc1_output"][a0:a1].cpu()
        sc_b = saved["fc1_output_scale"][a0:a1].float().cpu()
        assert torch.all((sc_b - sc_o).abs() <= bf16_ulp(sc_o * O.FP8_MAX) / O.FP8_MAX * 1.0001)
        same_scale = (sc_b == sc_o).repeat_interleave(O.FC1_SCALE_GROUP, dim=1)
        step = (e4m3_magnitude_index(codes_b) - e4m3_magnitude_index(codes_o)).abs()
        assert int(step[same_scale].max()) <= 1
        # (ii) the oracle's backward formula on the build's own save
        gu_b = O.dequantize_fc1(codes_b, sc_b)
        grad_act = O.bf16(O.bf16(dyr) @ w2e)
        scale = O.bf16(wr)[:, None]
        act_a, dact, v, dv = O.gated_act_grad(gu_b[:, :I], gu_b[:, I:], *ka[:4])
        dab_b = O.bf16(torch.cat([grad_act * dact * v * scale, grad_act * act_a * dv * scale], dim=1))
        got = g["grad_gate_up"][e].float().cpu()
        rel_b = max_rel(got, O.bf16(xr.T @ dab_b))
        rel_o = max_rel(got, O.bf16(xr.T @ own["dab"]))
        print(f"  expert {e}: {a1 - a0} rows, codes one step apart {int((step > 0).sum())}, scales moved "
              f"{int((sc_b != sc_o).sum())}; dW1 max-rel vs the oracle's own save {rel_o:.3e}, "
              f"vs the build's save {rel_b:.3e}", flush=True)
        assert rel_b <= 2e-2
