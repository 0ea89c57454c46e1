"""A packed chunked-prefill step (eager), after scheduler/mixed_module.py of the reference.

``upload`` builds the step's metadata exactly as the reference does
(scheduler/mixed_module.py:76-133): per-token slot ids, positions
``lens[slot] + offset``, pages ``block_table[slot, pos // P]`` and offsets
``pos % P``, ``cu_seqlens`` from the chunk lengths; ``forward`` runs the
model's decoder stack (each attention layer: token-mode KV append + varlen
mixed attention), advances ``lens`` by the chunk lengths and returns the
argmax token of each sequence's last row.  The reference's graph-captured
variants (full / piecewise) are not mirrored: the mixed step runs eagerly.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from ..attn.metadata import AttentionMetadata


class MixedModule:
    def __init__(self, model, kv_cache, token_count: int):
        self.model = model
        self.kv_cache = kv_cache
        self.token_count = token_count
        self.device = model.device
        self.metadata = AttentionMetadata(token_count=token_count, device=self.device, full_decode=False)
        self.lens = None
        self.last_logits = None  # (B, vocab) of the last forward
        self.static_input_ids = torch.zeros((1, token_count), device=self.device, dtype=torch.long)
        self.static_position_ids = torch.zeros((1, token_count), device=self.device, dtype=torch.long)

    def upload(self, prompts: list[list[int]], slot_ids: list[int]) -> int:
        lens_list = [len(p) for p in prompts]
        total_T = sum(lens_list)
        if total_T > self.token_count:
            raise ValueError(f"{total_T} tokens exceed the step's budget of {self.token_count}")
        dev = self.device
        lens = torch.tensor(lens_list, dtype=torch.long, device=dev)
        slots = torch.tensor(slot_ids, dtype=torch.long, device=dev)
        cu_seqlens = F.pad(lens.cumsum(0), (1, 0))
        ext_slots = torch.repeat_interleave(slots, lens, output_size=total_T)
        seq_off = torch.arange(total_T, device=dev) - torch.repeat_interleave(cu_seqlens[:-1], lens,
                                                                              output_size=total_T)
        pos = self.kv_cache.lens[ext_slots] + seq_off
        ids = torch.tensor([t for p in prompts for t in p], dtype=torch.long, device=dev)
        self.static_input_ids.zero_()
        self.static_position_ids.zero_()
        self.static_input_ids[0, :total_T] = ids
        self.static_position_ids[0, :total_T] = pos
        self.metadata.write_pages(self.kv_cache.block_table[ext_slots, pos // self.kv_cache.page_size])
        self.metadata.write_offsets(pos % self.kv_cache.page_size)
        self.metadata.slot_ids = slots
        self.metadata.cu_seqlens = cu_seqlens
        self.metadata.max_seqlen = max(lens_list) if lens_list else 0
        self.lens = lens
        return total_T

    def forward(self, prompts: list[list[int]], slot_ids: list[int]) -> list[int]:
        """Prefill (a chunk of) each prompt into its slot; returns each sequence's next token."""
        if not slot_ids:
            return []
        with torch.inference_mode():
            self.upload(prompts, slot_ids)
            # the whole token bucket runs, as in the reference: padding tokens
            # append to the reserved page 0 and lie outside every sequence
            hidden = self.model.model(input_ids=self.static_input_ids,
                                      position_ids=self.static_position_ids,
                                      kv_manager=self.kv_cache, use_cache=False,
                                      metadata=self.metadata).last_hidden_state
            self.kv_cache.mixed_advance(slot_ids=self.metadata.slot_ids, lens=self.lens)
            logits = self.model.lm_head(hidden[0, self.metadata.cu_seqlens[1:] - 1])
            self.last_logits = logits
            next_tokens = torch.argmax(logits, dim=-1)
            self.kv_cache.last_generated[self.metadata.slot_ids] = next_tokens
        return next_tokens.tolist()
