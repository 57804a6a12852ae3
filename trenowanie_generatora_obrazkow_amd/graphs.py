"""A fixed-shape layer step captured as one HIP graph and replayed.

Every hmoe entry point launches on the caller's current stream, allocates nothing itself (torch allocates the outputs
and workspaces) and never synchronises or reads data back, so a whole step -- router, dispatch, the GEMMs, combine, and
with autograd the full backward -- can be captured once and replayed: the replay launches the same kernels on the same
(static) tensors without the host work between them.  Nothing in the library records a hipMemsetAsync (counters and
scratch are written by the kernels themselves), so replays give the eager results bit for bit.

Usage (the tensors the step reads must stay the same objects; their contents may change between replays):

    def step():
        for p in params:
            p.grad = None                  # the captured backward then owns the gradient tensors
        out, _, _ = moe_swiglu(x, wr, wgu, wd, k)
        out.backward(dout)
        return out
    g = StepGraph(step)
    grads = [p.grad for p in params]       # the captured backward's gradient tensors
    out = g.replay()                       # same tensors every replay, now holding this replay's values
"""
from __future__ import annotations

import torch


class StepGraph:
    """Captures `fn` (no arguments) as a HIP graph after `warmup` eager calls on a side stream (torch's capture
    requirement: the allocator and lazily created state settle first).  Streams are created with the default
    priority."""

    def __init__(self, fn, warmup: int = 3):
        if not torch.cuda.is_available():
            raise RuntimeError("StepGraph needs a GPU")
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                fn()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.out = fn()
        torch.cuda.synchronize()

    def replay(self):
        """Launches the captured step on the current stream; returns what `fn` returned at capture (the same
        tensors, now holding this replay's values)."""
        self.graph.replay()
        return self.out
