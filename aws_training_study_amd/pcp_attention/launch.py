"""Launch-overhead path: a kernel call captured once into a HIP graph.

The reference's small configuration spends about 2.2 ms per call in host
launch and completion (README.md:105-107).  Here one call of the C ABI costs
a ctypes call plus argument checks; for small workloads that host time is
comparable to the kernel.  ``GraphedLaunch`` records a call sequence (the
history kernel, optionally the current-token step) into a HIP graph through
torch's graph capture; ``replay()`` then issues the whole recorded sequence
with one graph launch.  The recorded calls keep their tensors: update inputs
in place (``q.copy_(...)``, new pages through ``KVCacheWriter``) and read the
same output tensors after each replay.  The kernels record no memset nodes.
"""

from __future__ import annotations

from typing import Any, Callable


class GraphedLaunch:
    """``fn`` (a closure over fixed tensors) captured into a HIP graph.

    ``warmup`` eager calls run first on a side stream (they also allocate any
    workspace the call keeps, outside the capture).  ``result`` is what
    ``fn`` returned during capture; ``replay()`` re-runs the graph on the
    current stream and returns it.  ``fn`` is kept as long as the graph, and
    with it every tensor it closes over: the recorded kernels address their
    memory directly.
    """

    def __init__(self, fn: Callable[[], Any], warmup: int = 1):
        import torch

        self.fn = fn
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(max(warmup, 1)):
                fn()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.result = fn()

    def replay(self):
        self.graph.replay()
        return self.result

    __call__ = replay
