"""mm_route_noalloc (the routing entry point that allocates nothing: its
scratch is a library-owned device array) against mm_route with a caller
workspace, through the C ABI: bit-identical tables on two calls in a row,
the second smaller, with every output pre-filled with garbage; and sizes
beyond the scratch maximum are rejected before any launch."""

import pytest
import torch

from mega_moe import _lib
from mega_moe.runtime.routing import RouteTables

pytestmark = pytest.mark.gpu


def _tables(sel, E, with_w, fill):
    t = RouteTables(sel.numel(), E, sel.shape[1], sel.device, with_w)
    for name in ("counts", "offsets", "send_route", "send_token", "route_to_send"):
        getattr(t, name).fill_(fill)
    if with_w:
        t.weight_perm.fill_(float(fill))
    return t


def _args(sel, rw, t):
    return (_lib.ptr(sel), sel.numel(), sel.shape[1], t.num_experts, _lib.ptr(rw), _lib.ptr(t.counts),
            _lib.ptr(t.offsets), _lib.ptr(t.send_route), _lib.ptr(t.send_token), _lib.ptr(t.route_to_send),
            _lib.ptr(t.weight_perm))


def _check_equal(a, b, nvalid):
    assert torch.equal(a.counts, b.counts) and torch.equal(a.offsets, b.offsets)
    assert torch.equal(a.route_to_send, b.route_to_send)
    assert torch.equal(a.send_route[:nvalid], b.send_route[:nvalid])
    assert torch.equal(a.send_token[:nvalid], b.send_token[:nvalid])
    if a.weight_perm is not None:
        assert torch.equal(a.weight_perm[:nvalid], b.weight_perm[:nvalid])


def test_route_noalloc_matches_route_twice():
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = _lib.load()
    assert lib.mm_route_noalloc_scratch_bytes() == 4 << 20
    stream = _lib.stream_of(dev)
    g = torch.Generator().manual_seed(17)
    # first call: Kimi-scale routing (65536 routes, 896 experts, drops);
    # second: a smaller call whose tables must not inherit the first's
    for T, k, E in ((4096, 16, 896), (300, 4, 40)):
        sel = torch.randint(-2, E + 2, (T, k), generator=g, dtype=torch.int32).to(dev)
        rw = torch.rand(T, k, generator=g).to(dev)
        ref = _tables(sel, E, True, -7)
        ws = torch.empty(int(lib.mm_route_workspace_bytes(sel.numel(), E)), dtype=torch.uint8, device=dev)
        _lib.call("mm_route", *_args(sel, rw, ref), _lib.ptr(ws), ws.numel(), stream)
        got = _tables(sel, E, True, 12345)
        _lib.call("mm_route_noalloc", *_args(sel, rw, got), stream)
        torch.cuda.synchronize()
        nvalid = int(ref.offsets[-1])
        assert nvalid == int(((sel >= 0) & (sel < E)).sum())
        _check_equal(got, ref, nvalid)
        # without routing weights, too
        got2 = _tables(sel, E, False, 3)
        _lib.call("mm_route_noalloc", *_args(sel, None, got2), stream)
        torch.cuda.synchronize()
        _check_equal(got2, _strip(ref), nvalid)


def _strip(t):
    t.weight_perm = None
    return t


def test_route_noalloc_rejects_sizes_beyond_scratch():
    lib = _lib.load()
    dev = torch.device("cuda:0")
    sel = torch.zeros(1, 1, dtype=torch.int32, device=dev)
    t = _tables(sel, 1024, False, 0)
    huge = 4 << 20   # 4M routes x 1024 experts: 8 GiB of count table
    rc = lib.mm_route_noalloc(_lib.ptr(sel), huge, 1, 1024, None, _lib.ptr(t.counts), _lib.ptr(t.offsets),
                              _lib.ptr(t.send_route), _lib.ptr(t.send_token), _lib.ptr(t.route_to_send), None,
                              _lib.stream_of(dev))
    assert rc == -1 and b"scratch" in lib.mm_last_error()
