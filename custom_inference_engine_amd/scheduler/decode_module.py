"""One decode step of the whole model, captured in a hipGraph per batch bucket.

Mirrors scheduler/decode_module.py:8-107 of the reference: static ``(1, B)``
token and position buffers, a full-decode ``AttentionMetadata``, warmup runs
on a side stream, one graph capture of the step (the model forward — whose
attention layers run the fused KV append + paged decode — plus
``decode_advance``), then ``upload`` / ``replay`` / argmax per step.  The
reference compiles the forward with ``torch.compile`` before capture; here the
eager forward is captured as is (the attention path is already one HIP launch
per layer, and the rest of the layer is library GEMMs and elementwise ops).
"""
from __future__ import annotations

import torch

from ..attn.metadata import AttentionMetadata
from .slots import pad_slot_ids


class DecodeModule:
    def __init__(self, model, kv_cache, batch_size: int, pool=None, warmup_iters: int = 3):
        self.model = model
        self.batch_size = batch_size
        self.kv_cache = kv_cache
        device = model.device
        self.device = device

        self.metadata = AttentionMetadata(token_count=batch_size, device=device, full_decode=True)
        self.metadata.prepare_full_graph(batch_size)

        with torch.inference_mode():
            self.static_token = torch.zeros((1, batch_size), device=device, dtype=torch.long)
            self.static_position_ids = torch.zeros((1, batch_size), device=device, dtype=torch.long)

            side = torch.cuda.Stream(device=device)
            side.wait_stream(torch.cuda.current_stream(device))
            with torch.cuda.stream(side):
                for _ in range(max(1, warmup_iters)):
                    self._forward()
            torch.cuda.current_stream(device).wait_stream(side)
            torch.cuda.synchronize(device)

            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph, pool=pool):
                self.static_logits = self._forward().logits[0]
        self.warmup()

    def warmup(self) -> None:
        slot_ids = list(range(1, min(self.batch_size, self.kv_cache.n_slots - 1) + 1))
        self.forward(slot_ids)
        self.kv_cache.reset(slot_ids)

    def _forward(self):
        outputs = self.model(input_ids=self.static_token, position_ids=self.static_position_ids,
                             kv_manager=self.kv_cache, logits_to_keep=0, use_cache=False,
                             metadata=self.metadata)
        self.kv_cache.decode_advance(slot_ids=self.metadata.slot_ids)
        return outputs

    def upload(self, slot_ids: list[int]) -> None:
        padded = pad_slot_ids(slot_ids, self.batch_size, self.kv_cache.unused_idx)
        self.static_position_ids.copy_(self.kv_cache.lens[padded][None])
        self.static_token.copy_(self.kv_cache.last_generated[padded][None])
        self.metadata.write_slot_ids(slot_ids)

    def replay(self) -> torch.Tensor:
        self.graph.replay()
        return self.static_logits

    def forward(self, slot_ids: list[int]) -> list[int]:
        if not slot_ids:
            return []
        with torch.inference_mode():
            self.upload(slot_ids)
            logits = self.replay()
            next_tokens = torch.argmax(logits, dim=-1)[:len(slot_ids)]
            self.kv_cache.last_generated[slot_ids] = next_tokens
        return next_tokens.tolist()
