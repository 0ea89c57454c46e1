"""Host logic of the step modules (CPU): slot padding and page assignment."""
import pytest
import torch
from transformers import Qwen2Config

from custom_inference_engine_amd import KVStorage
from custom_inference_engine_amd.scheduler import assign_pages, pad_slot_ids


def test_pad_slot_ids_matches_reference_rule():
    assert pad_slot_ids([3, 1], 4, 0) == [3, 1, 0, 0]
    assert pad_slot_ids([1, 2], 2, 0) == [1, 2]
    with pytest.raises(ValueError):
        pad_slot_ids([1, 2, 3], 2, 0)


def test_assign_pages_writes_the_row_and_consumes_the_free_list():
    cfg = Qwen2Config(hidden_size=64, num_attention_heads=4, num_key_value_heads=2, num_hidden_layers=1)
    kv = KVStorage(cfg, max_cache_len=256, page_size=16, n_slots=3, device="cpu", dtype=torch.float16)
    free = list(range(1, kv.n_pages))
    assign_pages(kv, 2, 40, free)          # 3 pages
    assert kv.block_table[2, :3].tolist() == [15, 14, 13]
    assert kv.block_table[2, 3:].eq(0).all() and len(free) == 12
    with pytest.raises(ValueError):
        assign_pages(kv, 1, 16 * 13, free)   # 13 pages, 12 free
