"""Slot padding (scheduler/slots.py of the reference) and a page-assignment helper."""
from __future__ import annotations

import torch


def pad_slot_ids(slot_ids: list[int], batch_size: int, unused_slot: int) -> list[int]:
    """Pad ``slot_ids`` to ``batch_size`` with the reserved slot (scheduler/slots.py:1-12)."""
    missing = batch_size - len(slot_ids)
    if missing < 0:
        raise ValueError("more elements than batch size")
    return list(slot_ids) + [unused_slot] * missing


def assign_pages(kv_cache, slot: int, n_tokens: int, free_pages: list[int]) -> None:
    """Give ``slot`` enough pages from ``free_pages`` (popped from the end) for ``n_tokens``.

    Writes the slot's block-table row; the caller owns the free list (page 0
    is the reserved padding page and never handed out).
    """
    n = -(-n_tokens // kv_cache.page_size)
    if n > kv_cache.block_table.shape[1]:
        raise ValueError(f"{n_tokens} tokens need {n} pages, the row holds {kv_cache.block_table.shape[1]}")
    if n > len(free_pages):
        raise ValueError(f"{n} pages needed, {len(free_pages)} free")
    pages = [free_pages.pop() for _ in range(n)]
    row = torch.zeros(kv_cache.block_table.shape[1], dtype=torch.long)
    row[:n] = torch.tensor(pages, dtype=torch.long)
    kv_cache.block_table[slot].copy_(row.to(kv_cache.block_table.device))
