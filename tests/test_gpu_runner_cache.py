"""The in-process runner cache of einsum() (builder.py:887-902 rebuilds a
runner per call; here runners are cached, so eviction frees workspaces).
Runner workspaces come from torch's stream-ordered allocator: evicting a
runner must not synchronise the device (the reference's one-shot path frees
its workspace synchronously, builder.py:738-746), and a graph capture that
overflows the cache must keep every runner it used until the capture ends."""
import pytest
import torch

from pto_einsum import StageGraph, builder, einsum

pytestmark = pytest.mark.gpu

# Seven distinct contraction shapes, each needing a workspace (split-K
# partials or a staged output), against a cache of four.
SHAPES = [("ts,sp->tp", (64 + 8 * i, 1024), (1024, 64)) for i in range(4)] + \
         [("abc,cd->adb", (8, 6 + i, 40), (40, 12)) for i in range(3)]


@pytest.fixture
def small_cache(monkeypatch):
    builder.clear_runner_cache()
    monkeypatch.setattr(builder, "_RUNNER_CACHE_SIZE", 4)
    yield
    builder.clear_runner_cache()


def _operands(seed):
    g = torch.Generator().manual_seed(seed)
    return [(eq, torch.randn(s0, generator=g).cuda(), torch.randn(s1, generator=g).cuda()) for eq, s0, s1 in SHAPES]


def test_eviction_does_not_wait_for_the_device(small_cache):
    if not hasattr(torch.cuda, "_sleep"):
        pytest.skip("torch.cuda._sleep unavailable")
    ops = _operands(1)
    want = [torch.einsum(eq, a.double(), b.double()) for eq, a, b in ops]
    for eq, a, b in ops:  # build every runner once (JIT libraries on disk)
        einsum(eq, a, b)
    builder.clear_runner_cache()
    torch.cuda.synchronize()
    # A long kernel on another stream; evicting runners on this stream must
    # not wait for it.
    side = torch.cuda.Stream()
    done = torch.cuda.Event()
    with torch.cuda.stream(side):
        torch.cuda._sleep(1_500_000_000)
        done.record(side)
    got = [einsum(eq, a, b) for eq, a, b in ops]          # three evictions on the way
    assert len(builder._runners) == 4
    assert not done.query(), "an eviction waited for unrelated device work"
    torch.cuda.synchronize()
    for g_, w in zip(got, want):
        assert float((g_.double() - w).abs().max()) <= 1e-4 * max(1.0, float(w.abs().max()))


def test_capture_overflowing_the_cache(small_cache):
    ops = _operands(2)

    def stage():
        return [einsum(eq, a, b) for eq, a, b in ops]

    eager = [t.clone() for t in stage()]
    graph = StageGraph(stage)
    # During the capture no runner was evicted: all seven are still cached.
    assert len(builder._runners) == len(SHAPES)
    for rep in range(3):
        for eq_a_b in ops:  # new inputs, written in place
            eq_a_b[1].mul_(-1.0 if rep % 2 == 0 else -1.0)
        outs = graph.replay()
        torch.cuda.synchronize()
        now = [einsum(eq, a, b) for eq, a, b in ops]      # eager, trims the cache back
        torch.cuda.synchronize()
        for o, n in zip(outs, now):
            assert torch.equal(o, n)
    assert len(builder._runners) == 4
    del graph, eager
