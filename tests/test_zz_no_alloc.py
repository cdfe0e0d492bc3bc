"""cin_moe_route_noalloc (the route with a library-held scratch array instead of a
workspace argument) against cin_moe_route with a caller workspace, through the C ABI.

Two calls in a row share the GPU's scratch array; the second one is smaller, so it runs
over what the first left there.  A route that needs more scratch than the library holds
is rejected before any GPU work.  Captured in a HIP graph (after a first call outside the
capture has looked up the array's address), every replay equals the workspace route.
"""
import ctypes

import pytest
import torch

from cinnamon_amd import _lib
from oracle import fp8_oracle as orc

pytestmark = pytest.mark.gpu


def _zipf_ids(T, k, E, seed):
    g = torch.Generator().manual_seed(seed)
    p = torch.tensor([(e + 1) ** -1.1 for e in range(E)])
    return torch.multinomial(p.expand(T, E), k, replacement=False, generator=g)


def _route(idx, E, noalloc):
    lib = _lib.load()
    T, k = idx.shape
    dev = idx.device
    perm = torch.full((T * k,), -7, dtype=torch.int64, device=dev)
    inv = torch.full((T * k,), -7, dtype=torch.int32, device=dev)
    counts, starts, ends = (torch.full((E,), -7, dtype=torch.int64, device=dev) for _ in range(3))
    stream = _lib.stream_of(idx)
    outs = [_lib.ptr(t) for t in (perm, inv, counts, starts, ends)]
    if noalloc:
        rc = lib.cin_moe_route_noalloc(_lib.ptr(idx), T, k, E, *outs, stream)
    else:
        n = lib.cin_moe_route_workspace(T, k, E)
        ws = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
        rc = lib.cin_moe_route(_lib.ptr(idx), T, k, E, *outs, _lib.ptr(ws), n, stream)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    return perm.cpu(), inv.cpu(), counts.cpu(), starts.cpu(), ends.cpu()


@pytest.mark.parametrize("cases", [
    [(16384, 8, 32), (1000, 2, 17)],        # config 3's routing, then a smaller route
    [(4096, 8, 256), (77, 1, 5)],           # DeepSeek-V3's 256 experts, then a tiny one
])
def test_noalloc_route_equals_the_workspace_route(dev, cases):
    for i, (T, k, E) in enumerate(cases):
        idx = _zipf_ids(T, k, E, seed=T + E).to(dev)
        got = _route(idx, E, noalloc=True)
        want = _route(idx, E, noalloc=False)
        for a, b, name in zip(got, want, ("perm", "inv", "counts", "starts", "ends")):
            assert torch.equal(a, b), f"call {i} ({T}x{k}, E={E}): {name} differs"
        order, _, rc, rs, re_ = orc.moe_dispatch_ref(idx.cpu(), E)
        assert torch.equal(got[0], order) and torch.equal(got[2], rc)
        assert torch.equal(got[3], rs) and torch.equal(got[4], re_)


def test_noalloc_route_rejects_routes_beyond_its_scratch(dev):
    lib = _lib.load()
    T, k, E = 1 << 20, 8, 512        # needs 2 * 8192 * 512 = 8M int32 > 1M
    assert lib.cin_moe_route_workspace(T, k, E) > (1 << 20)
    small = torch.zeros(8, dtype=torch.int64, device=dev)
    p = _lib.ptr(small)
    rc = lib.cin_moe_route_noalloc(p, T, k, E, p, p, p, p, p, _lib.stream_of(small))
    assert rc == _lib.CIN_ERR_ARG
    assert "scratch" in _lib.last_error()
    assert isinstance(lib.cin_moe_route_noalloc, ctypes._CFuncPtr)


def test_noalloc_route_in_a_captured_graph(dev):
    """Warm the entry point once (its first call on a device looks up the scratch array's
    address), capture it in a torch.cuda.CUDAGraph, then replay the graph on new routing ids
    copied into its input buffer, with eager work and synchronizations between the replays:
    every replay's outputs equal cin_moe_route's on the same ids."""
    lib = _lib.load()
    T, k, E = 4096, 8, 64
    idx = _zipf_ids(T, k, E, seed=1).to(dev)
    perm = torch.empty(T * k, dtype=torch.int64, device=dev)
    inv = torch.empty(T * k, dtype=torch.int32, device=dev)
    counts, starts, ends = (torch.empty(E, dtype=torch.int64, device=dev) for _ in range(3))
    outs = [_lib.ptr(t) for t in (perm, inv, counts, starts, ends)]
    assert lib.cin_moe_route_noalloc(_lib.ptr(idx), T, k, E, *outs, _lib.stream_of(idx)) == 0
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib.cin_moe_route_noalloc(_lib.ptr(idx), T, k, E, *outs, _lib.stream_of(idx))
    assert rc == 0, _lib.last_error()
    for rep in range(4):
        new = _zipf_ids(T, k, E, seed=50 + rep).to(dev)
        idx.copy_(new)
        for t in (perm, inv, counts, starts, ends):
            t.fill_(-7)
        graph.replay()
        torch.cuda.synchronize()
        got = (perm.cpu(), inv.cpu(), counts.cpu(), starts.cpu(), ends.cpu())
        want = _route(new, E, noalloc=False)
        for a, b, name in zip(got, want, ("perm", "inv", "counts", "starts", "ends")):
            assert torch.equal(a, b), f"replay {rep}: {name} differs"
