"""GPU tests of stream use: concurrent calls on two caller streams, and HIP
graph capture of custom_kernel (the library's side stream joins the capture
through its event waits) replayed several times with eager work and
synchronisations between the replays, every replay checked bit for bit
against an eager call on the same input (the paths are deterministic).
"""
import sys

import pytest
import torch

from fastqr import custom_kernel

pytestmark = pytest.mark.gpu


def gaussian(batch, n, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn((batch, n, n), generator=g, dtype=torch.float32)


@pytest.mark.parametrize("n", [48, 150, 600, 2100])
def test_two_caller_streams_concurrently(cuda, n):
    print(f"[streams] n={n}", flush=True)
    sys.stdout.flush()
    batch = 2 if n > 1024 else 6
    a1, a2 = gaussian(batch, n, 11).to(cuda), gaussian(batch, n, 12).to(cuda)
    r1 = [t.clone() for t in custom_kernel(a1.clone())]
    r2 = [t.clone() for t in custom_kernel(a2.clone())]
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s1):
        h1, t1 = custom_kernel(a1)
    with torch.cuda.stream(s2):
        h2, t2 = custom_kernel(a2)
    torch.cuda.synchronize()
    assert torch.equal(h1, r1[0]) and torch.equal(t1, r1[1])
    assert torch.equal(h2, r2[0]) and torch.equal(t2, r2[1])


@pytest.mark.parametrize("n", [32, 150, 600])
def test_graph_capture_replays_match_eager(cuda, n):
    print(f"[graph] n={n}", flush=True)
    sys.stdout.flush()
    batch = 4
    a = gaussian(batch, n, 20).to(cuda)
    # warm-up on a side stream (library side stream, workspaces), as torch
    # recommends before capture
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        custom_kernel(a)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        h, tau = custom_kernel(a)
    for i in range(3):
        x = gaussian(batch, n, 100 + i).to(cuda)
        a.copy_(x)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        he, te = custom_kernel(x.clone())
        torch.cuda.synchronize()
        assert torch.equal(h, he), f"replay {i}: H differs from the eager call"
        assert torch.equal(tau, te), f"replay {i}: tau differs from the eager call"
