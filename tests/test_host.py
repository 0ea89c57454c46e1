"""Host-side logic that needs no GPU: metadata padding, KVStorage bookkeeping,
validation (mirroring the reference's asserts), op registration / fake impls,
the Qwen2 module swap, and the no-CPU-fallback rule."""
import pytest
import torch
from transformers import Qwen2Config, Qwen2ForCausalLM

import custom_inference_engine_amd as cie
from custom_inference_engine_amd.attn import core
from oracle import inputs


def _cfg(layers=2):
    return Qwen2Config(hidden_size=896, num_attention_heads=14, num_key_value_heads=2,
                       intermediate_size=256, num_hidden_layers=layers, vocab_size=128,
                       max_position_embeddings=512)


def test_metadata_padding_writers():
    m = cie.AttentionMetadata(token_count=6, full_decode=False, device="cpu")
    m.prepare_full_graph(4)
    m.write_slot_ids([3, 1])
    assert m.slot_ids.tolist() == [3, 1, 0, 0]
    m.write_cu_seqlens([0, 2, 5])
    assert m.cu_seqlens.tolist() == [0, 2, 5, 5, 5]  # padded sequences have zero rows
    m.write_pages([7, 7, 9])
    m.write_offsets([14, 15, 0])
    assert m.pages.tolist() == [7, 7, 9, 0, 0, 0] and m.offsets.tolist() == [14, 15, 0, 0, 0, 0]
    assert m.max_seqlen == 6 and m.full_decode is False
    with pytest.raises(ValueError):
        m.write_pages(list(range(7)))


def test_kvstorage_layout_and_bookkeeping():
    kv = cie.KVStorage(_cfg(), max_cache_len=100, page_size=16, n_slots=5, device="cpu",
                       dtype=torch.float16)
    assert kv.n_pages == 7 and kv.unused_idx == 0
    assert len(kv.keys) == 2 and kv.keys[0].shape == (7, 2, 16, 64)
    assert kv.keys[1].is_contiguous() and kv.keys[1].stride() == (2048, 1024, 64, 1)
    assert kv.block_table.shape == (5, 7) and kv.lens.dtype == torch.long
    kv.decode_advance(torch.tensor([2, 0, 3, 0]))
    assert kv.lens.tolist() == [0, 0, 1, 1, 0]  # slot 0 (padding) stays 0
    kv.mixed_advance(torch.tensor([2, 4]), torch.tensor([10, 3]))
    assert kv.lens.tolist() == [0, 0, 11, 1, 3]
    kv.block_table[2, :3] = torch.tensor([4, 5, 6])
    kv.reset([2])
    assert kv.lens[2] == 0 and kv.block_table[2].sum() == 0


def test_kv_append_has_no_cpu_fallback():
    kv = cie.KVStorage(_cfg(1), max_cache_len=64, page_size=16, n_slots=2, device="cpu",
                       dtype=torch.float16)
    k = torch.zeros(1, 1, 2, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="HIP device"):
        kv.decode_update(0, torch.tensor([1]), k, k)


def test_attention_has_no_cpu_fallback():
    case = inputs.make_case([10], seed=1)
    with pytest.raises(RuntimeError, match="HIP device"):
        cie.decode_gqa_attention(case.q, case.k_pool, case.v_pool, case.attended, case.slot_ids,
                                 case.block_table, num_programs=2)
    with pytest.raises(RuntimeError, match="HIP device"):
        cie.mixed_gqa_attention(case.q, case.k_pool, case.v_pool, 1, case.cu_seqlens, case.kv_lens,
                                case.slot_ids, case.block_table)


@pytest.mark.parametrize("mutate,match", [
    (lambda a: a.update(q=a["q"][:, :, :13]), "multiple"),                     # H_q % H_kv
    (lambda a: a.update(lens=a["lens"][:0]), "lens"),                          # lens shape
    (lambda a: a.update(block_table=a["block_table"][:, :-1]), "block_table"),  # width != n_pages
    (lambda a: a.update(q=a["q"].transpose(1, 2).contiguous().transpose(1, 2)), "contiguous"),
    (lambda a: a.update(q=a["q"].float()), "float16"),
])
def test_decode_validation_mirrors_reference_asserts(mutate, match):
    case = inputs.make_case([10, 20], seed=2)
    a = dict(q=case.q, k=case.k_pool, v=case.v_pool, lens=case.attended, slot_ids=case.slot_ids,
             block_table=case.block_table)
    mutate(a)
    with pytest.raises(AssertionError, match=match):
        cie.decode_gqa_attention(**a, num_programs=2)


def test_mixed_validation_mirrors_reference_asserts():
    case = inputs.make_case([10, 20], [3, 1], seed=3)
    with pytest.raises(AssertionError, match="cu_seqlens"):
        cie.mixed_gqa_attention(case.q, case.k_pool, case.v_pool, 3, case.cu_seqlens[:-1],
                                case.kv_lens, case.slot_ids, case.block_table)
    with pytest.raises(AssertionError, match="kv_lens"):
        cie.mixed_gqa_attention(case.q, case.k_pool, case.v_pool, 3, case.cu_seqlens,
                                case.kv_lens[:1], case.slot_ids, case.block_table)


def test_ops_registered_with_fake_impls():
    from torch._subclasses.fake_tensor import FakeTensorMode

    for name in ("gqa_decode_attention", "gqa_mixed_attention", "kv_append_decode", "kv_append_tokens",
                 "gqa_decode_append_attention"):
        assert hasattr(torch.ops.inference, name)
    case = inputs.make_case([10, 20], seed=4)
    attended = case.attended
    with FakeTensorMode() as mode:
        q = mode.from_tensor(case.q)
        k = mode.from_tensor(case.k_pool)
        out = torch.ops.inference.gqa_decode_attention(q, k, k, mode.from_tensor(attended),
                                                       mode.from_tensor(case.slot_ids),
                                                       mode.from_tensor(case.block_table))
        assert out.shape == case.q.shape and out.dtype == torch.float16
        out = torch.ops.inference.gqa_mixed_attention(
            q, k, k, 1, mode.from_tensor(case.cu_seqlens), kv_lens=mode.from_tensor(case.kv_lens),
            slot_ids=mode.from_tensor(case.slot_ids), block_table=mode.from_tensor(case.block_table))
        assert out.shape == case.q.shape
    schema = str(torch.ops.inference.kv_append_decode.default._schema)
    assert "!) k_cache" in schema and "!) v_cache" in schema and "!) k," not in schema
    schema = str(torch.ops.inference.gqa_decode_append_attention.default._schema)
    assert "!) k_cache" in schema and "!) v_cache" in schema and "!) q," not in schema


def test_default_split_policy():
    # about one split workgroup per CU (256 on MI355X)
    assert core.default_decode_splits(32, 2) == 4
    assert core.default_decode_splits(16, 2) == 8
    assert core.default_decode_splits(1, 2) == core.DECODE_MAX_SPLITS
    assert core.default_decode_splits(4096, 2) == 1
    # never past one workgroup per CU: 256 // 56 = 4 (not round(4.57) = 5)
    assert core.default_decode_splits(28, 2) == 4
    assert core.default_decode_splits(48, 2) == 2
    assert core.default_decode_splits(72, 2) == 1


def test_module_swap_and_fallback():
    model = Qwen2ForCausalLM(_cfg()).eval()
    cie.use_triton_attention(model)
    swapped = [m for m in model.modules() if isinstance(m, cie.TritonQwen2Attention)]
    assert len(swapped) == 2 and model._uses_triton_attention
    cie.use_triton_attention(model)  # idempotent
    assert len([m for m in model.modules() if isinstance(m, cie.TritonQwen2Attention)]) == 2
    attn = swapped[0]
    assert attn.qkv_weight.shape == (896 + 128 + 128, 896) and attn.qkv_sizes == [896, 128, 128]
    # no kv_manager: the wrapped HF module runs (attn/core.py:164-168)
    ids = torch.randint(0, 128, (1, 5))
    with torch.no_grad():
        out = model(input_ids=ids).logits
    assert out.shape == (1, 5, 128) and torch.isfinite(out).all()
    # kv_manager without metadata is an error (attn/core.py:170-174)
    hidden = torch.zeros(1, 1, 896)
    emb = model.model.rotary_emb(hidden, torch.zeros(1, 1, dtype=torch.long))
    with pytest.raises(ValueError, match="metadata"):
        attn(hidden, emb, kv_manager=object())
