"""Piecewise ``torch.compile`` backend (piecewise/backend.py:9-90 of the reference).

``get_piecewise_backend(out, pool)`` returns a backend that cuts a mixed
step's graph around its varlen attention calls (``utils.create_partition``).
The pieces without attention are captured in hipGraphs (allocations from the
shared ``pool``) on their first call and replayed afterwards; the attention
pieces run eagerly and write their output into ``out``, so the piece after
them always reads it from the same address.  Captured pieces are shared by
every graph the backend compiles (keyed by code and the inputs' layouts and
addresses), so the graphs compiled for different batch sizes of one token
bucket replay the same captured pieces.

The reference compiles each piece with inductor before capturing it; this
build captures the pieces' eager kernels (hipBLASLt GEMMs and ATen
elementwise kernels, with the paged-attention HIP kernels in between) and
generates no kernels, so no Triton code is involved.
"""
from __future__ import annotations

import torch

from .utils import create_partition, is_graph_piece, split


class _Replay:
    """A captured piece: replaying it refills the outputs it returned at capture."""

    def __init__(self, graph: torch.cuda.CUDAGraph, output) -> None:
        self.graph = graph
        self.output = output

    def __call__(self, *args):
        self.graph.replay()
        return self.output


def _capture(piece, pool, args) -> _Replay:
    dev = torch.cuda.current_device()
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        piece(*args)  # warm-up: lazy library state (hipBLASLt handles, workspaces)
    torch.cuda.current_stream(dev).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, pool=pool):
        output = piece(*args)
    graph.replay()  # this call's results
    return _Replay(graph, output)


def _eager_into(piece, out: torch.Tensor):
    def run(*args):
        out.copy_(piece(*args))
        return out
    return run


def _layout(arg):
    if isinstance(arg, torch.Tensor):
        return (tuple(arg.shape), tuple(arg.stride()), arg.dtype, arg.device, arg.data_ptr())
    return repr(arg)


def get_piecewise_backend(out: torch.Tensor, pool):
    """Backend for ``torch.compile`` (piecewise/backend.py:66-90 of the reference).

    ``out`` receives every attention piece's output, so it must hold the
    compiled step's attention output shape (``(1, T, H_q, D)``).  A captured
    piece is reused by a later compile only when its code and its inputs'
    shapes, strides and addresses all match: a hipGraph reads fixed addresses.
    """
    captured: dict = {}

    def backend(gm: torch.fx.GraphModule, example_inputs):
        pieces = split(gm, create_partition(gm))
        for name, piece in list(pieces.named_children()):
            if not is_graph_piece(piece):
                pieces.__dict__[name] = _eager_into(piece, out)
                continue

            def first_call(*args, _name=name, _piece=piece):
                key = (_piece.code,) + tuple(_layout(a) for a in args)
                replay = captured.get(key)
                if replay is None:
                    replay = captured[key] = _capture(_piece, pool, args)
                else:
                    replay.graph.replay()
                pieces.__dict__[_name] = replay
                return replay.output
            pieces.__dict__[name] = first_call
        return pieces

    return backend
