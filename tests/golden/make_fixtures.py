"""Writes tests/golden/layer_small.npz: seeded inputs of a small MoE layer and
the CPU oracle's outputs and gradients (bf16 stored as uint16 bit patterns).

    python tests/golden/make_fixtures.py
"""

import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import moe_oracle as O  # noqa: E402


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def main():
    T, H, I, E, k = 64, 256, 128, 4, 2
    g = torch.Generator().manual_seed(2024)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    sel = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
    sel[1, 0] = -1        # dropped routes
    sel[7, 1] = E
    rw = torch.softmax(torch.randn(T, k, generator=g), dim=-1)
    gate_up = (torch.randn(E, H, 2 * I, generator=g) * 0.1).to(torch.bfloat16)
    down = (torch.randn(E, H, I, generator=g) * 0.1).to(torch.bfloat16)
    dy = torch.randn(T, H, generator=g).to(torch.bfloat16)
    out, st = O.forward(x, sel, gate_up, down, rw)
    gr = O.backward(st, dy)
    tb = st["tables"]
    np.savez_compressed(
        os.path.join(os.path.dirname(os.path.abspath(__file__)), "layer_small.npz"),
        x=bits(x), selected=sel.numpy(), rw=rw.numpy(), gate_up=bits(gate_up), down=bits(down), dy=bits(dy),
        out=bits(out), grad_hidden=bits(gr["grad_hidden"]), grad_routing_weights=gr["grad_routing_weights"].numpy(),
        grad_gate_up=bits(gr["grad_gate_up"]), grad_fc2=bits(gr["grad_fc2"]),
        send_route=tb["send_route"], route_to_send=tb["route_to_send"], offsets=tb["offsets"])


if __name__ == "__main__":
    main()
