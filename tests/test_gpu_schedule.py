"""GPU: the persistent grid's tile queues.

Every eager launch pulls its tiles from device-side queue counters that the
last user of each queue resets to zero, in one of 1024 launch slots; a launch
recorded into a graph walks the same tile order statically, with no counters.
These tests check the contract that makes that safe: results never depend on
the slot, on what earlier launches left behind, on replays of captured graphs
(also concurrent ones), or on streams interleaving launches.  Each result is
compared bit for bit with an eager reference launch (same kernel, same inputs:
the tile order never changes a tile's arithmetic).
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(seed, shape, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(shape, generator=g).to(dtype).cuda() for _ in range(3))


def test_launch_slots_wrap(fa):
    """More launches than queue slots, mixing shapes (different queue sizes)."""
    qa, ka, va = _inputs(21, (2, 3, 300, 128))
    qb, kb, vb = _inputs(22, (1, 9, 130, 64), torch.float16)
    want_a = fa.attention(qa, ka, va, True, 0.09, return_lse=True)
    want_b = fa.attention(qb, kb, vb, False, 0.125, return_lse=True)
    for i in range(1100):
        if i % 2:
            got = fa.attention(qa, ka, va, True, 0.09, return_lse=True)
            want = want_a
        else:
            got = fa.attention(qb, kb, vb, False, 0.125, return_lse=True)
            want = want_b
        if i % 100 == 99:
            torch.cuda.synchronize()
            assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1]), i
    torch.cuda.synchronize()


@pytest.mark.parametrize("shape", [(2, 4, 700, 128), (1, 4, 700, 256)])
def test_graph_replays(fa, shape):
    """A captured launch replays with fresh queues (the last user resets them).
    D = 256 takes the kernel whose Q area is the launch's dynamic LDS."""
    q, k, v = _inputs(23, shape)
    want_o, want_l = fa.attention(q, k, v, True, 0.1, return_lse=True)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fa.attention(q, k, v, True, 0.1, return_lse=True)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out, lse = fa.attention(q, k, v, True, 0.1, return_lse=True)
    for rep in range(4):
        out.zero_()
        lse.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want_o) and torch.equal(lse, want_l), rep
        # eager work between replays takes other launch slots
        again = fa.attention(q, k, v, True, 0.1)
        torch.cuda.synchronize()
        assert torch.equal(again, want_o)


def test_concurrent_graph_replays(fa):
    """Captured launches use a static tile schedule (no queue counters): two graphs
    replayed concurrently on two streams, with eager launches on a third stream taking
    launch slots meanwhile, all match an eager reference bit for bit."""
    q, k, v = _inputs(26, (2, 8, 900, 128))
    want_o, want_l = fa.attention(q, k, v, True, 0.1, return_lse=True)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fa.attention(q, k, v, True, 0.1, return_lse=True)  # warm-up on a side stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graphs, outs = [], []
    for _ in range(2):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            outs.append(fa.attention(q, k, v, True, 0.1, return_lse=True))
        graphs.append(g)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream(), torch.cuda.Stream()]
    eager = []
    for rep in range(6):
        for o, l in outs:
            o.zero_()
            l.zero_()
        torch.cuda.synchronize()
        for g, st in zip(graphs, streams[:2]):
            with torch.cuda.stream(st):
                g.replay()
        with torch.cuda.stream(streams[2]):
            for _ in range(3):
                eager.append(fa.attention(q, k, v, True, 0.1))
        torch.cuda.synchronize()
        for o, l in outs:
            assert torch.equal(o, want_o) and torch.equal(l, want_l), rep
    for o in eager:
        assert torch.equal(o, want_o)


def test_two_streams(fa):
    """Launches interleaved on two streams use different slots and agree."""
    q, k, v = _inputs(24, (4, 8, 512, 128))
    want = fa.attention(q, k, v, True, 0.1)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = []
    for i in range(40):
        st = streams[i % 2]
        st.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(st):
            outs.append(fa.attention(q, k, v, True, 0.1))
    torch.cuda.synchronize()
    for o in outs:
        assert torch.equal(o, want)


@pytest.mark.parametrize("programs", ["1", "3", "8", "9", "100"])
def test_program_counts(fa, monkeypatch, programs):
    """Fewer programs than queues, odd counts, more programs than a queue's tiles."""
    q, k, v = _inputs(25, (3, 5, 390, 64), torch.float16)
    want = fa.attention(q, k, v, True, 0.1, return_lse=True)
    monkeypatch.setenv("PERSISTENT_PROGRAMS", programs)
    got = fa.attention(q, k, v, True, 0.1, return_lse=True)
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
