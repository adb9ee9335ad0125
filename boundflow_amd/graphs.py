"""Replay of launch-bound bound queries as HIP graphs.

A CROWN query on a small batch (C1: 576 bounds) is a few dozen short kernels;
issued one by one from Python its time is host launch overhead.  Capturing the
query once as a HIP graph (torch.cuda.CUDAGraph on ROCm) and replaying it
re-runs every kernel on the same device buffers with one launch.

Requirements of the captured function: device inputs that stay at the same
addresses, no host synchronization (the split-infeasibility check of the
forward trace is one: queries with splits or constraints are not capturable),
and no memset nodes (the library clears buffers with fill kernels).  Inputs may
be changed in place between replays (``copy_`` into the input box or center):
everything derived from them is recomputed inside the graph.  Operands derived
from the parameters (weight transposes, bias maps, packed conv weights) are
made once, before the capture, into storage the captured query keeps; a
parameter changed in place between replays has its operands remade into that
storage before the next replay.  The outputs of a replay live in the graph's
private memory pool and are overwritten by the next replay.
"""

from __future__ import annotations

from typing import Any, Callable

import torch


class CapturedQuery:
    """``fn()`` captured as a HIP graph; calling the object replays it and
    returns the (graph-owned) outputs of that replay."""

    def __init__(self, fn: Callable[[], Any], *, warmup: int = 2):
        from .crown import derived_scope
        # parameter-derived operands are made by the warm-up calls into a dict this
        # object keeps (never evicted, unlike the process-wide cache), so the graph
        # reads them instead of recomputing them on every replay
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with derived_scope() as self._derived, torch.cuda.stream(side):
            for _ in range(max(1, warmup)):
                fn()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with derived_scope(self._derived), torch.cuda.graph(self.graph):
            self.outputs = fn()
        torch.cuda.synchronize()

    def __call__(self) -> Any:
        from .crown import refresh_scope
        refresh_scope(self._derived)   # parameters changed in place since the last replay
        self.graph.replay()
        return self.outputs
