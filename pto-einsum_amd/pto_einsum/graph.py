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
eager call on the same inputs.  What must not run under capture -- building a
runner, creating its per-device workspace -- happens in the eager warm-up
calls that precede the capture.
"""
from __future__ import annotations

from typing import Any, Callable

import torch


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
            with torch.cuda.graph(self._graph):
                self.outputs = fn()
            torch.cuda.synchronize()

    def replay(self):
        """Reissue every captured launch; returns ``outputs``."""
        with torch.cuda.device(self.device):
            self._graph.replay()
        return self.outputs
