"""The drop-in attention layer under ``torch.compile(fullgraph=True)``, traced on
the CPU (no kernel runs): the reference compiles its decode step with
``fullgraph=True`` (scheduler/decode_module.py:33-44) and its piecewise backend
splits mixed steps at ``inference::gqa_mixed_attention`` nodes, reading their
``kv_lens`` keyword (piecewise/utils.py:5-7, 20).  Dynamo must therefore see
every paged-attention call as one opaque op (fake impls give it shapes), trace
the whole layer without a graph break, and keep ``kv_lens`` a keyword.

The recording backend below stops before execution: the ops run only on a
HIP device, and what is checked here is the graph a compile backend receives.
"""
import pytest
import torch
from transformers import Qwen2Config, Qwen2ForCausalLM

import custom_inference_engine_amd as cie

MIXED = torch.ops.inference.gqa_mixed_attention.default


class _Traced(Exception):
    pass


def _op_name(node) -> str:
    """Op of an FX node, with or without its overload (``.default``)."""
    return str(node.target).removesuffix(".default")


def _cfg():
    return Qwen2Config(hidden_size=896, num_attention_heads=14, num_key_value_heads=2,
                       intermediate_size=256, num_hidden_layers=1, vocab_size=128,
                       max_position_embeddings=512)


def layer_step(decode: bool, device="cpu", seed: int = 0):
    """One layer's inputs: 2 sequences in slots 1, 2 (4 rows for a mixed step),
    random weights, hidden states and pool contents."""
    cfg = _cfg()
    torch.manual_seed(seed)
    model = Qwen2ForCausalLM(cfg).eval().half().to(device)
    layer = cie.TritonQwen2Attention(model.model.layers[0].self_attn)
    kv = cie.KVStorage(cfg, max_cache_len=128, page_size=16, n_slots=3, device=device,
                       dtype=torch.float16)
    for pool in (kv.keys[0], kv.values[0]):
        pool.copy_(torch.randn(pool.shape) * 0.5)
    kv.block_table[1, :2] = torch.tensor([1, 2])
    kv.block_table[2, :2] = torch.tensor([3, 4])
    kv.lens[1], kv.lens[2] = 5, 9
    T = 2 if decode else 4
    meta = cie.AttentionMetadata(token_count=T, full_decode=decode, device=device)
    meta.prepare_full_graph(2)
    meta.write_slot_ids([1, 2])
    meta.write_cu_seqlens([0, 1, 2] if decode else [0, 3, 4])
    if not decode:
        meta.write_pages([1, 1, 1, 3])
        meta.write_offsets([5, 6, 7, 9])
    pos = (torch.tensor([[5, 9]]) if decode else torch.tensor([[5, 6, 7, 9]])).to(device)
    hidden = (torch.randn(1, T, cfg.hidden_size) * 0.5).half().to(device)
    cos, sin = model.model.rotary_emb(hidden, pos)
    return layer, kv, meta, hidden, cos, sin


def _trace(layer, kv, meta, hidden, cos, sin):
    graphs = []

    def backend(gm, example_inputs):
        graphs.append(gm)

        def run(*args):
            raise _Traced()
        return run

    torch._dynamo.reset()
    f = torch.compile(lambda h, c, s: layer(h, (c, s), kv_manager=kv, metadata=meta)[0],
                      backend=backend, fullgraph=True)
    with pytest.raises(_Traced):
        f(hidden, cos, sin)
    assert len(graphs) == 1
    return [n for n in graphs[0].graph.nodes if n.op == "call_function"]


@pytest.mark.parametrize("fuse_rope", [True, False], ids=["fused", "unfused"])
@pytest.mark.parametrize("decode", [True, False], ids=["decode", "mixed"])
def test_layer_traces_fullgraph(decode, fuse_rope):
    layer, kv, meta, hidden, cos, sin = layer_step(decode)
    layer.fuse_rope = fuse_rope
    nodes = _trace(layer, kv, meta, hidden, cos, sin)
    ops = {_op_name(n) for n in nodes if _op_name(n).startswith("inference.")}
    if decode:
        want = "inference.gqa_decode_qkv_rope_attention" if fuse_rope else \
            "inference.gqa_decode_append_attention"
        assert ops == {want}
    else:
        append = "inference.kv_append_tokens_qkv_rope" if fuse_rope else "inference.kv_append_tokens"
        assert ops == {append, "inference.gqa_mixed_attention"}
        mixed = [n for n in nodes if n.target is MIXED]
        assert len(mixed) == 1 and "kv_lens" in mixed[0].kwargs
        assert mixed[0].kwargs["max_seqlen"] == meta.max_seqlen


def test_two_launch_decode_branch_traces_fullgraph():
    """fuse_append = False: decode_update + the reference's decode op."""
    layer, kv, meta, hidden, cos, sin = layer_step(True)
    layer.fuse_rope, layer.fuse_append = False, False
    nodes = _trace(layer, kv, meta, hidden, cos, sin)
    ops = [_op_name(n) for n in nodes if _op_name(n).startswith("inference.")]
    assert ops == ["inference.kv_append_decode", "inference.gqa_decode_attention"]
