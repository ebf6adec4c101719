"""Replaying captured device work as one HIP graph.

A training or inference step on small inputs launches a few hundred short kernels; issuing them one by one from
Python costs more host time than the GPU needs to run them. Captured once into a HIP graph (torch.cuda.graph, whose
capture stream becomes the device's current stream), the step replays with one launch. The device's memory comes
from libomt_hip.so's allocator, so the capture also switches that allocator to a graph pool: every block the captured
kernels use stays reserved for the replays.

    g = Graph()
    with g.capture():
        loss = step()            # device work only: no host synchronization (.item(), printing) and no host copies
    g.replay()                   # runs the captured kernels again on the same memory; `loss` holds the new value

`graphed(fn)` wraps the usual recipe (warm-up calls on a side stream, then one capture). Optimizers stepped inside a
capture need capturable=True (their step counters then live on the device). Inputs that change between replays are
written into the captured tensors in place (`static_x.copy_(x)`).
"""

import contextlib

import torch

from omarchy_mac_torch.native import core


class Graph:
    """One captured sequence of device work and the memory it owns."""

    def __init__(self):
        self._graph = torch.cuda.CUDAGraph()
        self._torch_pool = torch.cuda.graph_pool_handle()  # memory of the ops delegated to torch's HIP kernels
        self._pool = core.graph_pool_create()              # memory of libomt_hip.so's allocator
        self._released = False

    @contextlib.contextmanager
    def capture(self):
        with torch.cuda.graph(self._graph, pool=self._torch_pool):
            core.graph_pool_begin(self._pool)
            try:
                yield self
            finally:
                core.graph_pool_end()

    def replay(self):
        if self._released:
            raise RuntimeError("omarchy_mac_torch.graphs.Graph: replay after release()")
        self._graph.replay()

    def release(self):
        """Frees the graph and returns its memory to the allocator; tensors created during capture must not be used
        afterwards."""
        if not self._released:
            self._graph.reset()
            core.graph_pool_release(self._pool)
            self._released = True


def graphed(fn, warmup=3):
    """Calls fn() `warmup` times eagerly on a side stream (plan tuning, allocator and optimizer state settle), then
    captures one call. Returns (replay, warmup_outputs): replay() re-runs the captured call and returns its outputs
    (the same tensors every time, refreshed by each replay). The warm-up calls do real work (an optimizer inside fn
    steps), their outputs are returned in order."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    outs = []
    with torch.cuda.stream(side):
        for _ in range(warmup):
            outs.append(fn())
    torch.cuda.current_stream().wait_stream(side)
    g = Graph()
    with g.capture():
        captured = fn()

    def replay():
        g.replay()
        return captured

    replay.graph = g
    return replay, outs
