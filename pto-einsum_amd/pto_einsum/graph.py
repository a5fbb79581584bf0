"""Replay a fixed sequence of einsum launches as one HIP graph.

Consumers such as the chunked GDN forward run several small contractions per
stage (reference: benchmarks/complex/gdn/einsum_gdn.py:94-372; the reference
names the per-stage launch overhead as its remaining cost,
IMPLEMENTATION.md:706-707).  At those sizes the host work of each call (the
Python checks, the output allocation, the ctypes call) takes longer than the
kernels.  ``StageGraph(fn)`` records every launch ``fn`` makes into one HIP
graph; ``replay()`` reissues them with no host work per launch.

What a replay reads and writes: exactly the device memory ``fn`` used during
capture.  Inputs are the tensors ``fn`` read (update them in place with
``copy_`` between replays); outputs are the tensors ``fn`` returned then
(``StageGraph.outputs``), overwritten by every replay.

The library's execution entry points are safe to capture: they launch kernels
on the caller's current stream and never allocate device memory, synchronise,
or clear memory with a memset (split-K partial sums are combined by a
reduction kernel in a fixed order), so every replay is bit-identical to an
eager call on the same inputs.  Runner workspaces are torch allocations
(allowed under capture); the graph keeps every einsum runner it captured alive,
so their workspaces outlive evictions from the runner cache, which pauses
while a capture runs.  Building runners (host-side code generation) is best
left to the eager warm-up calls that precede the capture.
"""
from __future__ import annotations

from typing import Any, Callable

import torch

from . import builder


class StageGraph:
    """``fn()`` captured once into a HIP graph and replayed on demand.

    ``warmup`` eager calls run first (they build runners and workspaces and
    must leave ``fn`` in a state where a further call launches work only).
    The capture runs on a side stream, as torch requires; ``replay()`` runs
    on the current stream.
    """

    def __init__(self, fn: Callable[[], Any], *, warmup: int = 2, device=None):
        if warmup < 1:
            raise ValueError("StageGraph: at least one eager warm-up call is required")
        self.device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        with torch.cuda.device(self.device):
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(warmup):
                    fn()
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            self._graph = torch.cuda.CUDAGraph()
            # Every einsum runner used in the capture is kept with the graph:
            # its workspace is part of what the replays read and write, so it
            # must outlive the runner cache's eviction of that runner.
            prev = builder._capture_pins
            builder._capture_pins = []
            try:
                with torch.cuda.graph(self._graph):
                    self.outputs = fn()
            finally:
                self._pinned = builder._capture_pins
                builder._capture_pins = prev
            torch.cuda.synchronize()

    def replay(self):
        """Reissue every captured launch; returns ``outputs``."""
        with torch.cuda.device(self.device):
            self._graph.replay()
        return self.outputs
