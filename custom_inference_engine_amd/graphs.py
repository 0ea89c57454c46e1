"""hipGraph capture shared by the step modules and the piecewise backend.

``StepGraph(fn)`` records one call of ``fn`` into a hipGraph and replays it.
Every capture here runs in inference mode: the first capture in a process
creates the random generators' capture state as tensors, and once those are
inference tensors (a capture in inference mode came first) a capture outside
inference mode fails when it updates them, so all captures keep one mode.
Everything ``fn`` touches must sit at fixed addresses from call to call (the
modules' static input blocks, the KV pool, the weights): a replay reruns the
recorded kernels with the recorded arguments.  Before the capture, ``fn`` runs
eagerly on a side stream (``warmup`` times) so that lazily created library
state — hipBLASLt handles, algorithm choices, workspaces, caching-allocator
blocks — exists before recording starts; the capture allocates from ``pool``
(a graph memory pool the caller may share between its graphs, so their
intermediates overlap in memory).  ``output`` is what the captured call
returned; every replay rewrites it in place.

``StepInputs`` is the other half of a replayable step: the per-step integer
inputs of a module live in one pinned host block and one device block with
the same layout, filled on the host and moved by one asynchronous copy.
"""
from __future__ import annotations

import numpy as np
import torch


class StepGraph:
    def __init__(self, fn, pool=None, warmup: int = 1, device=None) -> None:
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.device = dev
        main = torch.cuda.current_stream(dev)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(main)
        with torch.inference_mode():
            with torch.cuda.stream(side):
                for _ in range(max(1, warmup)):
                    fn()
            main.wait_stream(side)
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph, pool=pool):
                self.output = fn()
        self.replays = 0

    def replay(self):
        self.graph.replay()
        self.replays += 1
        return self.output


class StepInputs:
    """Named int64 vectors in one pinned host block and one device block.

    ``host(name)`` is a numpy view to fill; ``device(name)`` the matching
    device view (a fixed address, so a captured graph can read it);
    ``upload()`` enqueues one host-to-device copy of the whole block on the
    current stream.  The caller must not refill the host block before that
    copy has run (the step modules synchronize on each step's result).
    """

    def __init__(self, device, **lengths: int) -> None:
        total = sum(lengths.values())
        # pinned (hipHostMalloc) for an asynchronous copy to a HIP device
        pinned = torch.device(device).type == "cuda"
        self._host = torch.zeros(total, dtype=torch.long, pin_memory=pinned)
        self._host_np = self._host.numpy()
        self._dev = torch.zeros(total, dtype=torch.long, device=device)
        self._spans = {}
        start = 0
        for name, n in lengths.items():
            self._spans[name] = (start, start + n)
            start += n

    def host(self, name: str) -> np.ndarray:
        a, b = self._spans[name]
        return self._host_np[a:b]

    def device(self, name: str) -> torch.Tensor:
        a, b = self._spans[name]
        return self._dev[a:b]

    def upload(self) -> None:
        self._dev.copy_(self._host, non_blocking=True)
