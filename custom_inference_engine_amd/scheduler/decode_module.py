"""Whole-model decode steps replayed from one hipGraph per batch bucket.

Serves the decode steps of the reference's engine (one token per running
sequence; the reference's DecodeModule, scheduler/decode_module.py:8-107, is
the interface kept: constructor arguments, ``forward(slot_ids) -> next tokens``).

Design.  The only per-step input is the bucket's slot list (padded with the
reserved slot 0).  Everything else a step needs is already on the device and
is read inside the graph: the input token of sequence b is
``kv_cache.last_generated[slot_b]`` and its position is ``kv_cache.lens[slot_b]``
(two gathers recorded in the graph), the attention layers append and attend
through the fused decode kernel, ``decode_advance`` moves the lengths on, and
the LM head produces the bucket's logits.  The step's first launch is the
decode plan (``inference::gqa_decode_plan``): every layer's decode reads the
same slots, lengths and block-table rows, so their split counts (balanced by
length) and page ids are worked out once and each layer's launch starts one
memory round trip sooner.  A step is therefore: write the slot
ids into a pinned block, one asynchronous copy, one graph replay, then the
argmax and the ``last_generated`` update (kept out of the graph: argmax over a
151,936-wide vocabulary is a multi-block library reduction, and such library
kernels are not recorded) and one device-to-host copy of the tokens.

The capture's warm-up runs the step on the initial all-padding slot list, so it
touches only slot 0 and page 0 (reserved; ``decode_advance`` keeps slot 0's
length at zero): no real slot is used or has to be reset afterwards.
"""
from __future__ import annotations

import torch

from ..attn.core import gqa_decode_plan_op
from ..attn.metadata import AttentionMetadata
from ..graphs import StepGraph, StepInputs


class DecodeModule:
    def __init__(self, model, kv_cache, batch_size: int, pool=None, warmup_iters: int = 3):
        self.model = model
        self.kv_cache = kv_cache
        self.batch_size = batch_size
        self.device = model.device
        dev = self.device

        self.inputs = StepInputs(dev, slots=batch_size)
        self.inputs.host("slots")[:] = kv_cache.unused_idx
        self.inputs.upload()
        self.slots = self.inputs.device("slots")
        self.metadata = AttentionMetadata(token_count=batch_size, device=dev, full_decode=True)
        self.metadata.slot_ids = self.slots
        self.tokens = torch.zeros((batch_size,), dtype=torch.long, device=dev)
        self.positions = torch.zeros((batch_size,), dtype=torch.long, device=dev)
        with torch.inference_mode():
            self.step = StepGraph(self._step, pool=pool, warmup=warmup_iters, device=dev)
        self.logits = self.step.output  # (batch_size, vocab), rewritten by every replay

    def _step(self) -> torch.Tensor:
        kv = self.kv_cache
        # one plan for every layer's decode launch (their slots, lengths and
        # block-table rows are the step's): splits balanced by length, page
        # ids resolved once
        self.metadata.decode_plan = gqa_decode_plan_op(kv.keys[0], kv.lens, self.slots, kv.block_table)
        torch.index_select(kv.last_generated, 0, self.slots, out=self.tokens)
        torch.index_select(kv.lens, 0, self.slots, out=self.positions)
        hidden = self.model.model(input_ids=self.tokens[None], position_ids=self.positions[None],
                                  kv_manager=kv, use_cache=False,
                                  metadata=self.metadata).last_hidden_state
        kv.decode_advance(slot_ids=self.slots)
        return self.model.lm_head(hidden[0])

    def upload(self, slot_ids: list[int]) -> None:
        n = len(slot_ids)
        if n > self.batch_size:
            raise ValueError(f"{n} sequences do not fit the decode bucket of {self.batch_size}")
        host = self.inputs.host("slots")
        host[:n] = slot_ids
        host[n:] = self.kv_cache.unused_idx
        self.inputs.upload()

    def replay(self) -> torch.Tensor:
        return self.step.replay()

    def forward(self, slot_ids: list[int]) -> list[int]:
        n = len(slot_ids)
        if n == 0:
            return []
        with torch.inference_mode():
            self.upload(slot_ids)
            logits = self.replay()
            next_tokens = torch.argmax(logits[:n], dim=-1)
            self.kv_cache.last_generated[self.slots[:n]] = next_tokens
            return next_tokens.tolist()
