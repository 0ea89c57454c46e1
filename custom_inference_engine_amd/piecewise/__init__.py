"""Piecewise ``torch.compile`` backend for mixed steps (the reference's ``piecewise`` package)."""
from .backend import get_piecewise_backend
from .utils import create_partition, is_attention, is_graph_piece, split

__all__ = ["get_piecewise_backend", "create_partition", "is_attention", "is_graph_piece", "split"]
