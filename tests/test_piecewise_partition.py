"""The piecewise backend's graph cut (piecewise/utils.py:5-62 of the reference),
checked on the graph Dynamo traces for a 2-layer mixed step on the CPU (no
kernel runs: the recording backend stops before execution).

The cut must leave every ``inference::gqa_mixed_attention`` call in an
odd-numbered piece of its own, together with the gather of its ``kv_lens``,
and nothing that reads the batch's per-sequence tensors (``slot_ids``,
``cu_seqlens``) in the even-numbered pieces, which are replayed from
hipGraphs.
"""
import re

import pytest
import torch
from transformers import Qwen2Config, Qwen2ForCausalLM

from custom_inference_engine_amd import KVStorage, use_triton_attention
from custom_inference_engine_amd.piecewise import create_partition, is_attention, is_graph_piece, split
from custom_inference_engine_amd.scheduler import MixedModule, assign_pages


class _Traced(Exception):
    pass


def _traced_step(n_layers: int, chunks):
    cfg = Qwen2Config(hidden_size=896, num_attention_heads=14, num_key_value_heads=2,
                      intermediate_size=256, num_hidden_layers=n_layers, vocab_size=128,
                      max_position_embeddings=512)
    torch.manual_seed(0)
    model = Qwen2ForCausalLM(cfg).half().eval()
    use_triton_attention(model)
    kv = KVStorage(cfg, max_cache_len=256, page_size=16, n_slots=5, device="cpu", dtype=torch.float16)
    mod = MixedModule(model, kv, token_count=64)
    free = list(range(1, kv.n_pages))
    slots = list(range(1, len(chunks) + 1))
    for s in slots:
        assign_pages(kv, s, 40, free)
    graphs = []

    def backend(gm, example_inputs):
        graphs.append(gm)

        def run(*args):
            raise _Traced()
        return run

    torch._dynamo.reset()
    with torch.inference_mode():
        mod.upload([[1] * n for n in chunks], slots)
        mod._prepare()
        f = torch.compile(mod._forward, backend=backend, fullgraph=True, dynamic=False)
        with pytest.raises(_Traced):
            f()
    assert len(graphs) == 1
    return graphs[0]


@pytest.mark.parametrize("chunks", [[20, 5, 7], [9]], ids=["batch3", "batch1"])
@pytest.mark.parametrize("n_layers", [1, 3])
def test_partition_isolates_each_attention_call(n_layers, chunks):
    gm = _traced_step(n_layers, chunks)
    ids = create_partition(gm)
    attn = [n for n in gm.graph.nodes if is_attention(n)]
    assert len(attn) == n_layers
    for n in attn:
        assert ids[n] % 2 == 1
        gather = n.kwargs["kv_lens"]
        assert ids[gather] == ids[n]  # the kv_lens gather travels with its attention
    assert sorted({ids[n] for n in attn}) == [2 * i + 1 for i in range(n_layers)]

    pieces = dict(split(gm, ids).named_children())
    assert list(pieces) == [f"submod_{i}" for i in range(2 * n_layers + 1)]
    for i, (name, piece) in enumerate(pieces.items()):
        assert is_graph_piece(piece) == (i % 2 == 0)
        inputs = [p.name for p in piece.graph.nodes if p.op == "placeholder"]
        per_seq = [x for x in inputs if "slot_ids" in x or "cu_seqlens" in x or re.fullmatch(r"s\d+", x)]
        if i % 2 == 0:
            assert not per_seq, f"{name} reads per-sequence inputs {per_seq}"
        else:
            assert sum(is_attention(n) for n in piece.graph.nodes) == 1
