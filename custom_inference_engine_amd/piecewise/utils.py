"""Graph surgery for the piecewise backend (piecewise/utils.py:5-62 of the reference).

Dynamo hands the backend the FX graph of a whole mixed step.  Its varlen
attention calls (``inference::gqa_mixed_attention``) read the batch's
per-sequence tensors; everything between them (projections, norms, MLPs,
the KV append) reads only per-token tensors of the token bucket's shape.
The graph is cut around each attention node — together with the node that
gathers its ``kv_lens`` argument, which also reads the per-sequence
``slot_ids`` — into alternating pieces: the even-numbered ones hold no
attention and are replayed from hipGraphs, the odd-numbered ones run
eagerly.  Which nodes go where is the reference's rule, kept because the
pieces' inputs (what a recorded graph may read) follow from it.
"""
from __future__ import annotations

import torch
from torch.fx.passes.split_module import split_module

MIXED_ATTENTION = torch.ops.inference.gqa_mixed_attention.default


def is_attention(node) -> bool:
    return node.op == "call_function" and node.target is MIXED_ATTENTION


def create_partition(gm: torch.fx.GraphModule) -> dict:
    """Piece number of every compute node: each attention node and the
    producer of its ``kv_lens`` keyword share an odd number of their own; the
    nodes between two attentions share the even number between them."""
    piece, ids = 0, {}
    for node in gm.graph.nodes:
        if node.op in ("placeholder", "output"):
            continue
        if is_attention(node):
            piece += 1
            gather = node.kwargs["kv_lens"]
            if isinstance(gather, torch.fx.Node) and gather.op not in ("placeholder", "get_attr"):
                ids[gather] = piece
            ids[node] = piece
            piece += 1
        else:
            ids.setdefault(node, piece)
    return ids


def split(gm: torch.fx.GraphModule, ids: dict) -> torch.fx.GraphModule:
    return split_module(gm, None, lambda node: ids[node], keep_original_order=True)


def is_graph_piece(submod: torch.fx.GraphModule) -> bool:
    return not any(is_attention(n) for n in submod.graph.nodes)
