"""A packed chunked-prefill step, after scheduler/mixed_module.py of the reference.

``upload`` builds the step's metadata exactly as the reference does
(scheduler/mixed_module.py:76-133): per-token slot ids, positions
``lens[slot] + offset``, pages ``block_table[slot, pos // P]`` and offsets
``pos % P``, ``cu_seqlens`` from the chunk lengths; ``forward`` runs the
model's decoder stack (each attention layer: rope + token-mode KV append +
varlen mixed attention), advances ``lens`` by the chunk lengths and returns
the argmax token of each sequence's last row.

``MixedModule`` runs the step eagerly.  ``FullMixedModule`` captures the
decoder stack of one token bucket in a hipGraph, like the reference's
``FullMixedModule`` (scheduler/mixed_module.py:164-213): the batch is padded to
a fixed number of sequences with the reserved slot and zero-length chunks
(``cu_seqlens`` padded with its last value), pages / offsets with page 0, and
``max_seqlen`` is the token bucket; the varlen kernel plans its work on the
device, so padded sequences cost nothing.

``PiecewiseMixedModule`` is the reference's module for its larger token
buckets (scheduler/mixed_module.py:216-249): ``torch.compile`` of the stack
(``fullgraph=True``, ``dynamic=False``, the batch dimension of ``slot_ids`` and
``cu_seqlens`` marked dynamic) through the piecewise backend, which replays the
code between attention calls from hipGraphs and runs the varlen attention
eagerly into a shared buffer; the batch is not padded.  Here one full graph
per token bucket already covers every batch size, so the scheduler uses the
piecewise module only when asked to.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from ..attn.metadata import AttentionMetadata
from ..piecewise import get_piecewise_backend
from .slots import pad_slot_ids


class MixedModule:
    def __init__(self, model, kv_cache, token_count: int):
        self.model = model
        self.kv_cache = kv_cache
        self.token_count = token_count
        self.device = model.device
        self.metadata = AttentionMetadata(token_count=token_count, device=self.device, full_decode=False)
        self.lens = None
        self.last_logits = None  # (B, vocab) of the last forward
        with torch.inference_mode():
            self.static_input_ids = torch.zeros((1, token_count), device=self.device, dtype=torch.long)
            self.static_position_ids = torch.zeros((1, token_count), device=self.device, dtype=torch.long)

    # -- hooks: how the batch's per-sequence tensors reach the metadata, and how the stack runs

    def _pad(self, slot_ids: list[int]) -> list[int]:
        return list(slot_ids)

    def _write_batch(self, slots: torch.Tensor, cu_seqlens: torch.Tensor, lens: torch.Tensor) -> None:
        self.metadata.slot_ids = slots
        self.metadata.cu_seqlens = cu_seqlens
        self.lens = lens

    def _forward(self) -> torch.Tensor:
        return self.model.model(input_ids=self.static_input_ids, position_ids=self.static_position_ids,
                                kv_manager=self.kv_cache, use_cache=False,
                                metadata=self.metadata).last_hidden_state

    def replay(self) -> torch.Tensor:
        return self._forward()

    def warmup(self, n: int) -> None:
        """One real step through slots 1..n (then reset), as the reference's warm-up does
        (scheduler/mixed_module.py:41-47)."""
        slot_ids = list(range(1, n + 1))
        self.forward([[0] * (self.token_count // n) for _ in slot_ids], slot_ids)
        self.kv_cache.reset(slot_ids)

    # -- the step

    def upload(self, prompts: list[list[int]], slot_ids: list[int]) -> int:
        if len(prompts) != len(slot_ids):
            raise ValueError("len(prompts) must equal len(slot_ids).")
        padded = self._pad(slot_ids)
        lens_list = [len(p) for p in prompts] + [0] * (len(padded) - len(prompts))
        total_T = sum(lens_list)
        if total_T > self.token_count:
            raise ValueError(f"{total_T} tokens exceed the step's budget of {self.token_count}")
        dev = self.device
        lens = torch.tensor(lens_list, dtype=torch.long, device=dev)
        slots = torch.tensor(padded, dtype=torch.long, device=dev)
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
        self.metadata.max_seqlen = self.token_count
        self._write_batch(slots, cu_seqlens, lens)
        return total_T

    def forward(self, prompts: list[list[int]], slot_ids: list[int]) -> list[int]:
        """Prefill (a chunk of) each prompt into its slot; returns each sequence's next token."""
        if not slot_ids:
            return []
        with torch.inference_mode():
            self.upload(prompts, slot_ids)
            # the whole token bucket runs, as in the reference: padding tokens
            # append to the reserved page 0 and lie outside every sequence
            hidden = self.replay()
            self.kv_cache.mixed_advance(slot_ids=self.metadata.slot_ids, lens=self.lens)
            rows = self.metadata.cu_seqlens[1:len(slot_ids) + 1] - 1
            logits = self.model.lm_head(hidden[0, rows])
            self.last_logits = logits
            next_tokens = torch.argmax(logits, dim=-1)
            self.kv_cache.last_generated[self.metadata.slot_ids[:len(slot_ids)]] = next_tokens
        return next_tokens.tolist()


class FullMixedModule(MixedModule):
    """The decoder stack of one token bucket, captured in a hipGraph (see the module docstring)."""

    def __init__(self, model, kv_cache, batch_size: int, token_count: int, pool=None,
                 warmup_iters: int = 3):
        super().__init__(model, kv_cache, token_count)
        self.batch_size = batch_size
        self.metadata.prepare_full_graph(batch_size)
        with torch.inference_mode():
            self.static_lens = torch.zeros((batch_size,), dtype=torch.long, device=self.device)
            self.metadata.cu_seqlens.zero_()
            side = torch.cuda.Stream(device=self.device)
            side.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.stream(side):
                for _ in range(max(1, warmup_iters)):
                    self._forward()
            torch.cuda.current_stream(self.device).wait_stream(side)
            torch.cuda.synchronize(self.device)
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph, pool=pool):
                self.static_hidden = self._forward()
        self.lens = self.static_lens
        self.warmup(min(batch_size, kv_cache.n_slots - 1, token_count))

    def _pad(self, slot_ids: list[int]) -> list[int]:
        return pad_slot_ids(slot_ids, self.batch_size, self.kv_cache.unused_idx)

    def _write_batch(self, slots: torch.Tensor, cu_seqlens: torch.Tensor, lens: torch.Tensor) -> None:
        self.metadata.write_slot_ids(slots)
        self.metadata.write_cu_seqlens(cu_seqlens)
        self.static_lens.copy_(lens)

    def replay(self) -> torch.Tensor:
        self.graph.replay()
        return self.static_hidden


class PiecewiseMixedModule(MixedModule):
    """The stack compiled through the piecewise backend (see the module docstring).

    ``buffer`` (1, >= token_count, H_q, D) receives the attention outputs; it can
    be shared by the modules of every token bucket, as in the reference.
    """

    def __init__(self, model, kv_cache, token_count: int, buffer: torch.Tensor, pool=None):
        super().__init__(model, kv_cache, token_count)
        self.compiled = torch.compile(self._forward,
                                      backend=get_piecewise_backend(buffer[:, :token_count], pool),
                                      fullgraph=True, dynamic=False)
        self.warmup(min(kv_cache.n_slots - 1, token_count))
        self.warmup(1)

    def _write_batch(self, slots: torch.Tensor, cu_seqlens: torch.Tensor, lens: torch.Tensor) -> None:
        if len(slots) > 1:
            torch._dynamo.mark_dynamic(slots, 0)
            torch._dynamo.mark_dynamic(cu_seqlens, 0)
        super()._write_batch(slots, cu_seqlens, lens)

    def replay(self) -> torch.Tensor:
        return self.compiled()
