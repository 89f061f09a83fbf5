"""Process-group handling of FusedMoEForward on the CPU (gloo, two ranks).

As in the reference (ops/forward.py:78-243), ``ep_group=None`` reads the
default process group when torch.distributed is initialised. This build
keeps every expert on one GPU, so an expert-parallel world of two ranks is
rejected with NotImplementedError, while a one-rank group per process (each
GPU running its own full layer) is accepted. No device work happens here.
"""

import os
import socket

import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp


def _free_port():
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def _worker(rank, world, port, results):
    os.environ["MASTER_ADDR"] = "127.0.0.1"
    os.environ["MASTER_PORT"] = str(port)
    dist.init_process_group("gloo", rank=rank, world_size=world)
    try:
        import mega_moe
        kw = dict(max_tokens_per_rank=8, hidden_size=256, top_k=2, num_experts=4)
        out = {}
        try:
            mega_moe.FusedMoEForward(None, **kw)
            out["default_group"] = "accepted"
        except NotImplementedError as exc:
            out["default_group"] = "rejected" if "expert-parallel" in str(exc) else f"other: {exc}"
        solo = [dist.new_group([r]) for r in range(world)][rank]
        op = mega_moe.FusedMoEForward(solo, **kw)
        out["solo_group"] = (op.rank, op.world_size, op.experts_per_rank)
        try:
            mega_moe.FusedMoEForward(None, **dict(kw, num_experts=3))
            out["indivisible"] = "accepted"
        except ValueError:
            out["indivisible"] = "value_error"
        results[rank] = out
        dist.barrier()
    finally:
        dist.destroy_process_group()


def test_process_groups_two_ranks():
    world = 2
    port = _free_port()
    ctx = mp.get_context("spawn")
    with ctx.Manager() as m:
        results = m.dict()
        procs = [ctx.Process(target=_worker, args=(r, world, port, results)) for r in range(world)]
        for p in procs:
            p.start()
        for p in procs:
            p.join(timeout=120)
        for p in procs:
            if p.is_alive():
                p.kill()
                pytest.fail("worker did not finish")
            assert p.exitcode == 0
        res = dict(results)
    for r in range(world):
        assert res[r]["default_group"] == "rejected"
        assert res[r]["solo_group"] == (0, 1, 4)
        assert res[r]["indivisible"] == "value_error"
