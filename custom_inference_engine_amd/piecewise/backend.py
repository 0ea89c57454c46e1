"""Piecewise ``torch.compile`` backend (the reference's piecewise/backend.py:9-90).

``get_piecewise_backend(out, pool)`` returns a backend that cuts a mixed
step's graph around its varlen attention calls (``utils.create_partition``).
The pieces without attention are recorded into hipGraphs (``StepGraph``,
allocations from the shared ``pool``) on their first call and replayed
afterwards; the attention pieces run eagerly and write their output into
``out``, so the piece after them always reads it from the same address.

The reference compiles each piece with inductor before capturing it; this
build records the pieces' eager kernels (hipBLASLt GEMMs and ATen elementwise
kernels, with the paged-attention HIP kernels in between) and generates no
kernels, so no Triton code is involved.  The backend counts what it does
(``compiles``: graphs handed to it; ``piece_replays``: replays of recorded
pieces), so a caller can check that its steps run compiled.
"""
from __future__ import annotations

import torch

from ..graphs import StepGraph
from .utils import create_partition, is_graph_piece, split


class _GraphPiece:
    """A piece without attention: recorded on its first call, replayed after."""

    def __init__(self, piece, pool, stats) -> None:
        self.piece = piece
        self.pool = pool
        self.stats = stats
        self.graph: StepGraph | None = None

    def __call__(self, *args):
        if self.graph is None:
            # the inputs are the step's static buffers or earlier pieces' recorded
            # outputs: the same addresses on every call
            self.graph = StepGraph(lambda: self.piece(*args), pool=self.pool)
        self.stats.piece_replays += 1
        return self.graph.replay()


def _eager_into(piece, out: torch.Tensor):
    def run(*args):
        out.copy_(piece(*args))
        return out
    return run


def get_piecewise_backend(out: torch.Tensor, pool):
    """Backend for ``torch.compile`` (piecewise/backend.py:66-90 of the reference).

    ``out`` receives every attention piece's output, so it must hold the
    compiled step's attention output shape (``(1, T, H_q, D)``).
    """

    def backend(gm: torch.fx.GraphModule, example_inputs):
        backend.compiles += 1
        pieces = split(gm, create_partition(gm))
        for name, piece in list(pieces.named_children()):
            if is_graph_piece(piece):
                pieces.__dict__[name] = _GraphPiece(piece, pool, backend)
            else:
                pieces.__dict__[name] = _eager_into(piece, out)
        return pieces

    backend.compiles = 0
    backend.piece_replays = 0
    return backend
