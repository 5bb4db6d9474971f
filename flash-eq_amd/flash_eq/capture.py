"""Capture of a whole training step (forward, loss, backward) in one HIP graph.

The library launches every kernel on the caller's current stream, allocates its
workspaces through PyTorch's caching allocator and clears memory with kernels
(no hipMemsetAsync), so a step built from its ops records into a graph and
replays with none of the host work (Python, autograd, launch calls) of an
eager step.  Ops that synchronise with the host (``.item()``, host copies)
cannot be captured and raise during capture.
"""
from __future__ import annotations

from typing import Callable, Iterable

import torch


def capture_step(step: Callable[[], torch.Tensor], leaves: Iterable[torch.Tensor],
                 warmup: int = 3):
    """Records ``step`` (which runs forward, loss and backward and returns the
    loss) into a ``torch.cuda.CUDAGraph``.

    ``leaves``: the tensors whose ``.grad`` the step writes.  Their gradients are
    reset to None before the warmup runs and before capture, so the captured
    backward writes (rather than accumulates) them: after each ``replay()`` they
    hold that step's gradients.  Returns (graph, loss tensor of the graph)."""
    leaves = list(leaves)

    def clear():
        for t in leaves:
            t.grad = None

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(warmup):
            clear()
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    clear()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        loss = step()
    return graph, loss
