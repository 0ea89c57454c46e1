"""Packed chunked-prefill / decode steps over the paged pool.

Serves the mixed steps of the reference's engine: a batch of sequences, each
feeding a chunk of new tokens (a prompt piece, or one decode token), packed
into one token bucket.  The public surface is the reference's
(scheduler/mixed_module.py:10-249: ``MixedModule(model, kv_cache,
token_count)``, ``FullMixedModule(..., batch_size, token_count, pool)``,
``PiecewiseMixedModule(..., token_count, buffer, pool)``, and
``forward(prompts, slot_ids) -> next token per sequence``); the design below
is this build's own.

Design.  A step's host inputs are three fixed-size int64 vectors in one pinned
block (``StepInputs``): the batch's slot ids and chunk lengths, padded to the
module's batch capacity with slot 0 and length 0, and the packed token ids,
padded to the token bucket with 0.  One asynchronous copy moves them.
Everything else is derived on the device by ``_prepare`` (fixed shapes, in
place into static buffers, so it can be recorded in a graph): ``cu_seqlens``
by a cumulative sum of the lengths; the sequence of each packed row by a
binary search in ``cu_seqlens``; its position ``lens[slot] + offset in its
chunk``, page ``block_table[slot, pos // page_size]`` and in-page offset; rows
past the batch's tokens get slot 0, position 0, page 0, offset 0 (the
reserved padding targets).  Padded sequences have zero query rows, which the
varlen kernel skips at no cost (it plans its work on the device), so one
token bucket serves every batch size.  After the decoder stack, ``_advance``
moves each slot's length on by its chunk and ``_logits`` applies the LM head
to each sequence's last row; the argmax and the ``last_generated`` update
run after the step, as in the decode module.

Three ways to run the same step:
  * ``MixedModule``: everything eagerly.
  * ``FullMixedModule``: ``_prepare``, the decoder stack, ``_advance`` and
    ``_logits`` recorded in one hipGraph per token bucket (``StepGraph``);
    its warm-up runs on the all-padding inputs, which touch only slot 0 and
    page 0.
  * ``PiecewiseMixedModule``: the decoder stack compiled with
    ``torch.compile(fullgraph=True)`` through the piecewise backend (graph
    pieces between eagerly run attention calls); ``_prepare``, ``_advance``
    and ``_logits`` run eagerly.  All inputs have fixed shapes, so each token
    bucket compiles exactly once (no dynamic dimensions).
"""
from __future__ import annotations

import contextlib

import torch

from ..attn.core import gqa_mixed_plan_op
from ..attn.metadata import AttentionMetadata
from ..graphs import StepGraph, StepInputs
from ..piecewise import get_piecewise_backend


class MixedModule:
    def __init__(self, model, kv_cache, token_count: int, batch_size: int | None = None):
        self.model = model
        self.kv_cache = kv_cache
        self.token_count = token_count
        self.batch_size = batch_size or max(1, kv_cache.n_slots - 1)
        self.device = model.device
        dev, B, T = self.device, self.batch_size, token_count

        self.inputs = StepInputs(dev, slots=B, chunk_lens=B, tokens=T)
        self.slots = self.inputs.device("slots")
        self.chunk_lens = self.inputs.device("chunk_lens")
        self.tokens = self.inputs.device("tokens")
        self.inputs.host("slots")[:] = kv_cache.unused_idx
        self.inputs.upload()
        self.cu_seqlens = torch.zeros((B + 1,), dtype=torch.long, device=dev)
        self.positions = torch.zeros((T,), dtype=torch.long, device=dev)
        self.rows = torch.arange(T, dtype=torch.long, device=dev)
        self.metadata = AttentionMetadata(token_count=T, device=dev, full_decode=False)
        self.metadata.slot_ids = self.slots
        self.metadata.cu_seqlens = self.cu_seqlens
        self.metadata.max_seqlen = T
        self.last_logits = None  # (n, vocab) of the last forward

    # -- the step, in pieces

    def _prepare(self) -> None:
        """cu_seqlens, positions, pages and offsets from (slots, chunk_lens)."""
        kv, B = self.kv_cache, self.batch_size
        torch.cumsum(self.chunk_lens, 0, out=self.cu_seqlens[1:])
        seq = torch.searchsorted(self.cu_seqlens[1:], self.rows, right=True)
        live = seq < B
        seq.clamp_(max=B - 1)
        slot = torch.where(live, self.slots[seq], kv.unused_idx)
        pos = torch.where(live, kv.lens[slot] + (self.rows - self.cu_seqlens[seq]), 0)
        self.positions.copy_(pos)
        self.metadata.pages.copy_(torch.where(live, kv.block_table[slot, pos // kv.page_size], 0))
        self.metadata.offsets.copy_(pos % kv.page_size)
        # one plan for every layer's mixed attention: the step's sequences are
        # the same for all of them (the lengths advance after the step).  (A
        # step prepared on the CPU — traced, never run — has none.)
        if kv.keys[0].is_cuda:
            T = self.token_count
            self.metadata.mixed_plan = gqa_mixed_plan_op(
                kv.keys[0], self.cu_seqlens, kv.lens[self.slots], self.slots, kv.block_table, T, T,
                self.model.config.num_attention_heads)

    def _forward(self) -> torch.Tensor:
        return self.model.model(input_ids=self.tokens[None], position_ids=self.positions[None],
                                kv_manager=self.kv_cache, use_cache=False,
                                metadata=self.metadata).last_hidden_state

    def _advance(self) -> None:
        self.kv_cache.mixed_advance(slot_ids=self.slots, lens=self.chunk_lens)

    def _logits(self, hidden: torch.Tensor) -> torch.Tensor:
        last = (self.cu_seqlens[1:] - 1).clamp(min=0)
        return self.model.lm_head(hidden[0, last])

    def _step(self) -> torch.Tensor:
        self._prepare()
        hidden = self._forward()
        self._advance()
        return self._logits(hidden)

    def run(self) -> torch.Tensor:
        """The step on the uploaded inputs; (batch_size, vocab) logits."""
        return self._step()

    # -- host side

    def upload(self, prompts: list[list[int]], slot_ids: list[int]) -> int:
        if len(prompts) != len(slot_ids):
            raise ValueError("len(prompts) must equal len(slot_ids).")
        n = len(slot_ids)
        if n > self.batch_size:
            raise ValueError(f"{n} sequences do not fit the step's batch of {self.batch_size}")
        lens = [len(p) for p in prompts]
        total = sum(lens)
        if total > self.token_count:
            raise ValueError(f"{total} tokens exceed the step's budget of {self.token_count}")
        slots, chunk_lens, tokens = (self.inputs.host(k) for k in ("slots", "chunk_lens", "tokens"))
        slots[:n] = slot_ids
        slots[n:] = self.kv_cache.unused_idx
        chunk_lens[:n] = lens
        chunk_lens[n:] = 0
        tokens[:total] = [t for p in prompts for t in p]
        tokens[total:] = 0
        self.inputs.upload()
        return total

    def forward(self, prompts: list[list[int]], slot_ids: list[int]) -> list[int]:
        """Feed each sequence its chunk; returns each sequence's next token (argmax of
        its last row)."""
        n = len(slot_ids)
        if n == 0:
            return []
        with torch.inference_mode():
            self.upload(prompts, slot_ids)
            logits = self.run()[:n]
            self.last_logits = logits
            next_tokens = torch.argmax(logits, dim=-1)
            self.kv_cache.last_generated[self.slots[:n]] = next_tokens
            return next_tokens.tolist()


class FullMixedModule(MixedModule):
    """The whole step of one token bucket replayed from a hipGraph."""

    def __init__(self, model, kv_cache, batch_size: int, token_count: int, pool=None,
                 warmup_iters: int = 3):
        super().__init__(model, kv_cache, token_count, batch_size=batch_size)
        with torch.inference_mode():
            self.step = StepGraph(self._step, pool=pool, warmup=warmup_iters, device=self.device)

    def run(self) -> torch.Tensor:
        return self.step.replay()


class PiecewiseMixedModule(MixedModule):
    """The decoder stack compiled through the piecewise backend.

    ``buffer`` (1, >= token_count, H_q, D) receives the attention outputs; the
    modules of several token buckets may share it.  ``backend`` exposes how
    many graphs it compiled and how many captured pieces it replayed.
    """

    # Each bucket's module compiles the same ``_forward`` code once; the
    # compiles all happen in the constructors (fixed shapes), under this limit.
    RECOMPILE_LIMIT = 64

    def __init__(self, model, kv_cache, token_count: int, buffer: torch.Tensor, pool=None,
                 batch_size: int | None = None):
        super().__init__(model, kv_cache, token_count, batch_size=batch_size)
        self.backend = get_piecewise_backend(buffer[:, :token_count], pool)
        self.compiled = torch.compile(self._forward, backend=self.backend, fullgraph=True,
                                      dynamic=False)
        with self._compile_limits(), torch.inference_mode():
            self._prepare()  # the all-padding inputs: slot 0 and page 0 only
            self.compiled()

    @classmethod
    def _compile_limits(cls):
        dynamo = torch._dynamo.config
        limits = {"recompile_limit": max(dynamo.recompile_limit, cls.RECOMPILE_LIMIT)}
        if hasattr(dynamo, "accumulated_recompile_limit"):
            limits["accumulated_recompile_limit"] = max(dynamo.accumulated_recompile_limit,
                                                        cls.RECOMPILE_LIMIT)
        return dynamo.patch(**limits) if hasattr(dynamo, "patch") else contextlib.nullcontext()

    def _step(self) -> torch.Tensor:
        self._prepare()
        hidden = self.compiled()
        self._advance()
        return self._logits(hidden)
