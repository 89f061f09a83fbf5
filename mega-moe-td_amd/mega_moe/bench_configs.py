"""Case registry and seeded synthetic inputs for the benchmark configurations.

Plays the role of the reference's CaseSpec registry (config/_shapes.py:21-85)
for the five layer configurations this build is measured on. Inputs are
synthetic: x ~ N(0, 1), expert weights ~ N(0, 0.02), routing as described per
case. Weights are returned in the operator's layouts:
``gate_up`` [E, H, 2I] contiguous (= cat(W_gate, W_up) along the last dim) and
``down`` [E, H, I] as the transposed view of a natural W_down [E, I, H].
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class CaseSpec:
    name: str
    tokens: int
    hidden: int
    inter: int
    experts: int
    top_k: int
    routing: str          # "softmax_topk" | "uniform_distinct" | "zipf"
    backward: bool
    dtype: str = "bf16"
    zipf_s: float = 1.2

    @property
    def routes(self) -> int:
        return self.tokens * self.top_k

    def fwd_flops(self) -> float:
        return 6.0 * self.routes * self.hidden * self.inter

    def bwd_flops(self) -> float:
        return 12.0 * self.routes * self.hidden * self.inter

    def weight_bytes(self) -> float:
        return 6.0 * self.experts * self.hidden * self.inter


CASES = {
    "toy": CaseSpec("toy", 512, 256, 512, 8, 2, "softmax_topk", True, dtype="fp32"),
    "e32": CaseSpec("e32", 4096, 4096, 1536, 32, 8, "uniform_distinct", False),
    "qwen": CaseSpec("qwen", 8192, 2048, 768, 128, 8, "softmax_topk", True),
    "kimi": CaseSpec("kimi", 4096, 7168, 2048, 896, 16, "softmax_topk", True),
    "skew": CaseSpec("skew", 16384, 4096, 1536, 32, 8, "zipf", True),
    # the Kimi-scale layer at the reference's larger per-rank token counts
    "kimi8k": CaseSpec("kimi8k", 8192, 7168, 2048, 896, 16, "softmax_topk", True),
    "kimi16k": CaseSpec("kimi16k", 16384, 7168, 2048, 896, 16, "softmax_topk", True),
    # DeepSeek-V3-like layer: 256 experts, top-8, 128 rows per expert on average
    "dsv3": CaseSpec("dsv3", 4096, 7168, 2048, 256, 8, "softmax_topk", True),
}


def make_routing(spec: CaseSpec, gen: torch.Generator):
    """(selected [T, k] int32, routing_weights [T, k] fp32) on the CPU."""
    T, E, k = spec.tokens, spec.experts, spec.top_k
    if spec.routing == "softmax_topk":
        logits = torch.randn(T, E, generator=gen)
        probs = torch.softmax(logits, dim=-1)
        w, idx = torch.topk(probs, k, dim=-1)
        w = w / w.sum(dim=-1, keepdim=True)
    elif spec.routing == "uniform_distinct":
        idx = torch.rand(T, E, generator=gen).argsort(dim=1)[:, :k]
        w = torch.softmax(torch.randn(T, k, generator=gen), dim=-1)
    elif spec.routing == "zipf":
        p = (torch.arange(E, dtype=torch.float64) + 1.0).pow(-spec.zipf_s)
        p = (p / p.sum()).float()
        idx = torch.multinomial(p.expand(T, E), k, replacement=False, generator=gen)
        w = torch.softmax(torch.randn(T, k, generator=gen), dim=-1)
    else:
        raise ValueError(spec.routing)
    return idx.to(torch.int32).contiguous(), w.float().contiguous()


def make_inputs(spec: CaseSpec, device="cpu", seed: int = 1234, tokens: int | None = None,
                weight_scale: float = 0.02):
    """Seeded inputs; large tensors are drawn on `device` in expert chunks.

    Returns dict(x, selected, rw, gate_up, down, dy).
    """
    T = spec.tokens if tokens is None else tokens
    s = spec if tokens is None else CaseSpec(spec.name, T, spec.hidden, spec.inter, spec.experts, spec.top_k,
                                             spec.routing, spec.backward, spec.dtype, spec.zipf_s)
    gen = torch.Generator(device="cpu").manual_seed(seed)
    selected, rw = make_routing(s, gen)
    dev = torch.device(device)
    dgen = torch.Generator(device=dev).manual_seed(seed + 1)
    bf = torch.bfloat16
    x = torch.randn(T, s.hidden, generator=dgen, device=dev).to(bf)
    dy = torch.randn(T, s.hidden, generator=dgen, device=dev).to(bf)
    E, H, inter = s.experts, s.hidden, s.inter
    gate_up = torch.empty(E, H, 2 * inter, dtype=bf, device=dev)
    down_nat = torch.empty(E, inter, H, dtype=bf, device=dev)
    chunk = max(1, (1 << 28) // (H * inter * 4))
    for e0 in range(0, E, chunk):
        e1 = min(E, e0 + chunk)
        gate_up[e0:e1] = (torch.randn(e1 - e0, H, 2 * inter, generator=dgen, device=dev) * weight_scale).to(bf)
        down_nat[e0:e1] = (torch.randn(e1 - e0, inter, H, generator=dgen, device=dev) * weight_scale).to(bf)
    return dict(x=x, selected=selected.to(dev), rw=rw.to(dev), gate_up=gate_up, down=down_nat.transpose(1, 2),
                dy=dy)
