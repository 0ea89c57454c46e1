"""Per-forward attention metadata with the reference's ``AttentionMetadata`` surface.

Mirrors attn/metadata.py:3-55: ``slot_ids (B,)``, ``cu_seqlens (B+1,)``,
``pages (T,)``, ``offsets (T,)`` (all int64), ``max_seqlen`` = the token-count
bucket, ``full_decode``.  The writers keep shapes fixed for graph replay by
padding: slot ids and pages / offsets with 0 (slot 0 and page 0 are the
reserved padding targets) and cu_seqlens with its last value (so padded
sequences have zero query rows).
"""
from __future__ import annotations

import torch


class AttentionMetadata:
    def __init__(self, token_count: int, full_decode: bool, device: torch.device):
        self.device = device
        self.slot_ids = None
        self.cu_seqlens = None
        self.pages = torch.zeros((token_count,), dtype=torch.long, device=device)
        self.offsets = torch.zeros((token_count,), dtype=torch.long, device=device)
        self.max_seqlen = token_count
        self.full_decode = full_decode
        # a decode step's plan (inference::gqa_decode_plan), made once per
        # step by the step module and read by every layer; None: unplanned
        self.decode_plan = None
        # a mixed step's plan (inference::gqa_mixed_plan), likewise
        self.mixed_plan = None

    def prepare_full_graph(self, batch_size: int) -> None:
        self.slot_ids = torch.zeros((batch_size,), dtype=torch.long, device=self.device)
        self.cu_seqlens = torch.zeros((batch_size + 1,), dtype=torch.long, device=self.device)

    @staticmethod
    def _write(dst: torch.Tensor, values, pad) -> None:
        values = torch.as_tensor(values, dtype=torch.long, device=dst.device)
        n = len(values)
        if n > dst.shape[0]:
            raise ValueError(f"{n} values do not fit a buffer of {dst.shape[0]}")
        dst[:n] = values
        dst[n:] = pad(values)

    def write_slot_ids(self, ids) -> None:
        self._write(self.slot_ids, ids, lambda v: 0)

    def write_cu_seqlens(self, cu_seqlens) -> None:
        self._write(self.cu_seqlens, cu_seqlens, lambda v: v[-1])

    def write_pages(self, pages) -> None:
        self._write(self.pages, pages, lambda v: 0)

    def write_offsets(self, offsets) -> None:
        self._write(self.offsets, offsets, lambda v: 0)
