"""Paged GQA attention host functions, ``torch.library`` ops and the Qwen2 drop-in.

Same surface as the reference's attn/core.py:
  * ``decode_gqa_attention`` (attn/core.py:13-66) — split-KV decode, one query
    token per sequence; ``num_programs`` is the KV split count.
  * ``mixed_gqa_attention`` (attn/core.py:69-111) — varlen causal attention for
    packed chunked-prefill + decode batches.
  * ops ``inference::gqa_decode_attention`` / ``inference::gqa_mixed_attention``
    (attn/core.py:119-137): functional (``mutates_args=()``), with fake impls so
    ``torch.compile(fullgraph=True)`` traces through them.
  * ``TritonQwen2Attention`` / ``replace_attention`` / ``use_triton_attention``
    (attn/core.py:139-250).  The class keeps the reference's name so callers
    switch by import; it runs the gfx950 HIP kernels, not Triton.

The Triton launch knobs (``BLOCK_N``, ``BLOCK_M``, ``num_warps``, ``wrap``) are
accepted and ignored.  Validation mirrors the reference's asserts and raises
``AssertionError`` with the same conditions (never stripped by ``-O``).
Outputs are allocated with ``torch.empty`` on the current stream (under graph
capture they come from the graph pool), split partials likewise; the decode
kernels' arrival counters are one persistent, self-cleaning buffer per device
(``split_counters``).
The decode op also has a fused form, ``inference::gqa_decode_append_attention``,
that performs ``KVStorage.decode_update`` and the decode in one launch, and
the drop-in goes one step further by default: from the fused QKV projection's
output, ``inference::gqa_decode_qkv_rope_attention`` does the QKV split, RoPE,
the append and the decode in one launch, and ``inference::kv_append_tokens_qkv_rope``
does the split, RoPE and ``KVStorage.mixed_update`` of a mixed step in one.
"""
from __future__ import annotations

import threading
from typing import Optional

import torch
from transformers.models.qwen2.modeling_qwen2 import Qwen2Attention, apply_rotary_pos_emb

from .. import _native

# Decode kernel geometry: one split = one workgroup; the default split count
# keeps the grid at one workgroup per CU or fewer (MI355X: 256 CUs).
DECODE_DEFAULT_CUS = 256
DECODE_MAX_SPLITS = 64


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise AssertionError(msg)


def _index(t: torch.Tensor) -> torch.Tensor:
    if t.dtype != torch.int64 or not t.is_contiguous():
        t = t.to(torch.int64).contiguous()
    return t


def _block_table(bt: torch.Tensor) -> torch.Tensor:
    if bt.dtype != torch.int64 or bt.stride(1) != 1:
        bt = bt.to(torch.int64).contiguous()
    return bt


_ctr_lock = threading.Lock()
_ctr_cache: dict[int, torch.Tensor] = {}
_ctr_retired: list[torch.Tensor] = []


def _device_index(dev) -> int:
    dev = torch.device(dev)
    return dev.index if dev.index is not None else torch.cuda.current_device()


def split_counters(dev: torch.device, n: int) -> torch.Tensor:
    """The device's persistent split-arrival counters (zeroed once, kept zero by the kernels).

    The decode and mixed kernels' counters (arrival words, then as many stale
    words) must be zero before a call and are left zero by it, so one buffer
    serves every stream-ordered call on a device, graph replays included,
    without a clearing launch.  Calls that can overlap in time (different
    streams) must pass their own zeroed ``counters``; a kernel that finds a
    stale word raises ``CIE_ERRBIT_SPLIT`` in ``err``.  Replaced buffers stay
    alive: a captured graph may still point at them.
    """
    idx = _device_index(dev)
    with _ctr_lock:
        buf = _ctr_cache.get(idx)
        if buf is None or buf.numel() < n:
            if buf is not None:
                _ctr_retired.append(buf)
            buf = torch.zeros(max(n, 4096), dtype=torch.int32, device=torch.device("cuda", idx))
            _ctr_cache[idx] = buf
        return buf


def reset_split_counters(dev: torch.device) -> None:
    """Zero the device's persistent split counters (a fill kernel on the current stream).

    Needed only after a call raised ``CIE_ERRBIT_SPLIT``: a stale word inside
    ``[0, n_splits)`` cannot be told apart from live arrivals, so the kernels
    cannot be trusted to have cleaned it.  Stream-ordered like the calls."""
    idx = _device_index(dev)
    with _ctr_lock:
        buf = _ctr_cache.get(idx)
    if buf is not None:
        # the buffer may have been created under inference mode (captured steps)
        with torch.inference_mode():
            buf.zero_()


def _split_buffers(lib, dev, B, H_q, H_kv, D, P, counters):
    partials = torch.empty(lib.cie_paged_decode_partials_bytes(B, H_q, D, P), dtype=torch.uint8,
                           device=dev)
    if counters is None:
        counters = split_counters(dev, 2 * B * H_kv)
    _require(counters.dtype == torch.int32 and counters.numel() >= 2 * B * H_kv, "counters too small")
    return partials, counters


PLAN_WORDS_PER_WORKGROUP = 8 + 4 * 64  # descriptor + its 4 waves' page ids (int32)


def decode_plan(k_cache, lens, slot_ids, block_table, append: bool = True, num_programs=None,
                err=None) -> torch.Tensor:
    """One decode step's plan, made once and used by every layer's planned decode.

    The slot ids, lengths and block-table rows of a step are the same for all
    of its layers, so each sequence's attended length (``lens[slot] + 1`` with
    ``append``, else ``lens[b]``), its split count (balanced by length over
    the grid) and every workgroup's page ids are worked out once here; a
    layer's planned launch then reads its descriptor and page ids in one
    memory round trip.  ``num_programs`` (splits per sequence) sizes the grid
    at ``B * H_kv * num_programs`` workgroups; by default about one per CU.
    Returns an int32 tensor; pass it as ``plan=`` to the decode functions of
    the same step (same ``append`` mode, block table and lengths)."""
    N_PAGES, H_kv, PAGE_SIZE, _ = k_cache.shape
    B = slot_ids.shape[0]
    _require(N_PAGES == block_table.shape[1], "block_table width must equal n_pages")
    dev = _native.require_device(k_cache, lens, slot_ids, block_table)
    lens, slot_ids, block_table = _index(lens), _index(slot_ids), _block_table(block_table)
    lib = _native.load()
    P = int(num_programs) if num_programs else 0
    n_wg = lib.cie_paged_decode_plan_workgroups(max(B, 1), H_kv, P)
    _require(n_wg > 0, "num_programs outside [1, the kernel's split limit]")
    plan = torch.empty(n_wg * PLAN_WORDS_PER_WORKGROUP, dtype=torch.int32, device=dev)
    if B == 0:
        return plan
    _native.check(
        lib.cie_paged_decode_plan(
            plan.data_ptr(), lens.data_ptr(), slot_ids.data_ptr(), block_table.data_ptr(), B, H_kv,
            PAGE_SIZE, N_PAGES, block_table.stride(0), block_table.shape[1], lens.shape[0] if append
            else block_table.shape[0], int(bool(append)), n_wg, _native.ptr(err), _native.stream_handle(dev),
        ),
        "cie_paged_decode_plan",
    )
    return plan


def _plan_workgroups(plan: torch.Tensor) -> int:
    _require(plan.dtype == torch.int32 and plan.is_contiguous() and plan.dim() == 1
             and plan.numel() % PLAN_WORDS_PER_WORKGROUP == 0, "plan must come from decode_plan")
    return plan.numel() // PLAN_WORDS_PER_WORKGROUP


def _planned_buffers(lib, dev, B, H_q, H_kv, D, n_wg, counters):
    partials = torch.empty(lib.cie_paged_decode_planned_partials_bytes(n_wg, H_q, H_kv, D),
                           dtype=torch.uint8, device=dev)
    if counters is None:
        counters = split_counters(dev, 2 * B * H_kv)
    _require(counters.dtype == torch.int32 and counters.numel() >= 2 * B * H_kv, "counters too small")
    return partials, counters


def _cu_count(dev: torch.device | None) -> int:
    if dev is not None and dev.type == "cuda":
        return torch.cuda.get_device_properties(dev).multi_processor_count
    return DECODE_DEFAULT_CUS


def default_decode_splits(batch: int, h_kv: int, dev: torch.device | None = None) -> int:
    """KV splits per (sequence, kv head): the most that keep the grid at one
    workgroup per CU or fewer.  A grid past that (rounding 256 / 56 up to 5
    splits at B = 28, say) puts two workgroups on some CUs, and those set the
    call: 13.5 against 10.5 us at B = 28, 17.2 against 13.3 at B = 48."""
    units = max(1, batch * h_kv)
    return max(1, min(DECODE_MAX_SPLITS, _cu_count(dev) // units))


def _check_pool(q, k, v):
    _require(k.dim() == 4 and k.shape == v.shape, "K/V pools must be (n_pages, H_kv, page_size, D)")
    _require(
        k.stride() == v.stride() and k.stride(3) == 1 and k.stride(2) == q.shape[-1],
        "K/V pools need identical strides with dense (page_size, D) rows",
    )
    _require(q.dtype == torch.float16 and k.dtype == torch.float16 and v.dtype == torch.float16,
             "q and the K/V pools must be float16")


def decode_gqa_attention(q, k, v, lens, slot_ids, block_table, num_programs=None,
                         BLOCK_N=64, num_warps=4, wrap=None, err=None, counters=None, plan=None):
    """Paged GQA decode: ``o[0, b, h] = softmax(q[0, b, h] K^T / sqrt(D)) V`` over ``lens[b]`` tokens.

    q: (1, B, H_q, D) fp16 contiguous; k, v: (n_pages, H_kv, page_size, D);
    lens (B,) = attended lengths; slot_ids (B,); block_table (n_slots, n_pages).
    """
    total_T, H_q, D = q.shape[1:]
    N_PAGES, H_kv, PAGE_SIZE, _ = k.shape
    B = slot_ids.shape[0]
    _require(H_q % H_kv == 0, "H_q must be a multiple of H_kv")
    _require(tuple(lens.shape) == (B,), "lens must be (B,)")
    _require(N_PAGES == block_table.shape[1], "block_table width must equal n_pages")
    _require(total_T == B, "decode takes one query token per sequence")
    _require(q.is_contiguous(), "q must be contiguous")
    _check_pool(q, k, v)
    dev = _native.require_device(q, k, v, lens, slot_ids, block_table)
    lens, slot_ids, block_table = _index(lens), _index(slot_ids), _block_table(block_table)
    P = int(num_programs) if num_programs else default_decode_splits(B, H_kv, dev)
    _require(P >= 1, "num_programs must be >= 1")

    lib = _native.load()
    o = torch.empty_like(q)
    if B == 0:
        return o
    if plan is not None:  # a step's plan (decode_plan with append=False)
        n_wg = _plan_workgroups(plan)
        partials, counters = _planned_buffers(lib, dev, B, H_q, H_kv, D, n_wg, counters)
        _native.check(
            lib.cie_paged_decode_planned(
                o.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), plan.data_ptr(),
                block_table.data_ptr(), partials.data_ptr(), counters.data_ptr(), B, H_q, H_kv, D,
                PAGE_SIZE, N_PAGES, k.stride(0), k.stride(1), block_table.stride(0),
                block_table.shape[1], n_wg, _native.ptr(err), _native.stream_handle(dev),
            ),
            "cie_paged_decode_planned",
        )
        return o
    _require(P <= lib.cie_paged_decode_max_splits(), "num_programs above the kernel's split limit")
    partials, counters = _split_buffers(lib, dev, B, H_q, H_kv, D, P, counters)
    _native.check(
        lib.cie_paged_decode(
            o.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
            lens.data_ptr(), slot_ids.data_ptr(), block_table.data_ptr(), partials.data_ptr(),
            counters.data_ptr(),
            B, H_q, H_kv, D, PAGE_SIZE, N_PAGES, k.stride(0), k.stride(1),
            block_table.stride(0), block_table.shape[1], block_table.shape[0], P,
            _native.ptr(err), _native.stream_handle(dev),
        ),
        "cie_paged_decode",
    )
    return o


def decode_append_gqa_attention(q, k_cache, v_cache, k, v, lens, slot_ids, block_table,
                                num_programs=None, err=None, counters=None, plan=None):
    """KV append of the new token + paged GQA decode in one launch.

    Same result as ``KVStorage.decode_update`` (kv_cache/storage.py:87-122)
    followed by ``decode_gqa_attention(..., lens[slot_ids] + 1, ...)``
    (attn/core.py:200-215): the pools gain k[b] / v[b] at position
    ``lens[slot_ids[b]]`` and each sequence attends that many tokens plus one.
    ``lens`` is the pool's per-slot length (n_slots,), not advanced here.
    """
    total_T, H_q, D = q.shape[1:]
    N_PAGES, H_kv, PAGE_SIZE, _ = k_cache.shape
    B = slot_ids.shape[0]
    _require(H_q % H_kv == 0, "H_q must be a multiple of H_kv")
    _require(N_PAGES == block_table.shape[1], "block_table width must equal n_pages")
    _require(total_T == B, "decode takes one query token per sequence")
    _require(q.is_contiguous(), "q must be contiguous")
    _check_pool(q, k_cache, v_cache)
    dev = _native.require_device(q, k_cache, v_cache, k, v, lens, slot_ids, block_table)
    kr, vr = _as_rows(k, H_kv, D), _as_rows(v, H_kv, D)
    _require(kr.shape[0] == B and vr.shape[0] == B, "one new K/V row per sequence")
    _require(kr.dtype == torch.float16 and vr.dtype == torch.float16, "new K/V must be float16")
    lens, slot_ids, block_table = _index(lens), _index(slot_ids), _block_table(block_table)
    P = int(num_programs) if num_programs else default_decode_splits(B, H_kv, dev)
    _require(P >= 1, "num_programs must be >= 1")

    lib = _native.load()
    o = torch.empty_like(q)
    if B == 0:
        return o
    if plan is not None:  # a step's plan (decode_plan with append=True)
        n_wg = _plan_workgroups(plan)
        partials, counters = _planned_buffers(lib, dev, B, H_q, H_kv, D, n_wg, counters)
        _native.check(
            lib.cie_paged_decode_append_planned(
                o.data_ptr(), q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                kr.data_ptr(), vr.data_ptr(), kr.stride(0), kr.stride(1), vr.stride(0), vr.stride(1),
                plan.data_ptr(), block_table.data_ptr(), partials.data_ptr(), counters.data_ptr(),
                B, H_q, H_kv, D, PAGE_SIZE, N_PAGES, k_cache.stride(0), k_cache.stride(1),
                block_table.stride(0), block_table.shape[1], n_wg,
                _native.ptr(err), _native.stream_handle(dev),
            ),
            "cie_paged_decode_append_planned",
        )
        return o
    _require(P <= lib.cie_paged_decode_max_splits(), "num_programs above the kernel's split limit")
    partials, counters = _split_buffers(lib, dev, B, H_q, H_kv, D, P, counters)
    _native.check(
        lib.cie_paged_decode_append(
            o.data_ptr(), q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
            kr.data_ptr(), vr.data_ptr(), kr.stride(0), kr.stride(1), vr.stride(0), vr.stride(1),
            lens.data_ptr(), slot_ids.data_ptr(), block_table.data_ptr(), partials.data_ptr(),
            counters.data_ptr(),
            B, H_q, H_kv, D, PAGE_SIZE, N_PAGES, k_cache.stride(0), k_cache.stride(1),
            block_table.stride(0), block_table.shape[1], lens.shape[0], P,
            _native.ptr(err), _native.stream_handle(dev),
        ),
        "cie_paged_decode_append",
    )
    return o


def _qkv_rows(qkv: torch.Tensor, width: int) -> torch.Tensor:
    """(1, T, width) fused projection output -> (T, width) rows the kernels can read."""
    _require(qkv.dim() == 3 and qkv.shape[0] == 1 and qkv.shape[2] == width,
             f"qkv must be (1, T, {width})")
    _require(qkv.dtype == torch.float16, "qkv must be float16")
    rows = qkv[0]
    if rows.stride(1) != 1 or rows.stride(0) % 8 or rows.data_ptr() % 16:
        rows = rows.contiguous()
    return rows


def _rope_rows(t: torch.Tensor, n: int, d: int) -> torch.Tensor:
    """cos / sin of shape (1, n, d) or (n, d) -> (n, d) rows, 16-byte aligned."""
    _require(t.dtype == torch.float16, "cos / sin must be float16")
    rows = t.reshape(-1, d)
    _require(rows.shape[0] == n, "one cos / sin row per token")
    if rows.stride(1) != 1 or rows.stride(0) % 8 or rows.data_ptr() % 16:
        rows = rows.contiguous()
    return rows


def decode_qkv_rope_gqa_attention(qkv, cos, sin, k_cache, v_cache, lens, slot_ids, block_table,
                                  num_heads: int, num_programs=None, err=None, counters=None,
                                  plan=None):
    """Decode step from the fused QKV projection output, one launch.

    ``qkv`` (1, B, (H_q + 2·H_kv)·D) is ``F.linear(hidden, qkv_weight, qkv_bias)``
    of TritonQwen2Attention (attn/core.py:181-184); ``cos`` / ``sin`` (1, B, D)
    are the step's rotary tables.  Same result as splitting q / k / v,
    ``apply_rotary_pos_emb`` (attn/core.py:193-198, computed in fp32 and
    rounded once to fp16) and ``decode_append_gqa_attention``: the pools gain
    the rotated k and v rows at ``lens[slot_ids[b]]``; returns o (1, B, H_q, D).
    """
    N_PAGES, H_kv, PAGE_SIZE, D = k_cache.shape
    H_q = int(num_heads)
    B = slot_ids.shape[0]
    _require(H_q % H_kv == 0, "H_q must be a multiple of H_kv")
    _require(N_PAGES == block_table.shape[1], "block_table width must equal n_pages")
    rows = _qkv_rows(qkv, (H_q + 2 * H_kv) * D)
    _require(rows.shape[0] == B, "decode takes one query token per sequence")
    q_like = rows.new_empty((1, B, H_q, D))
    _check_pool(q_like, k_cache, v_cache)
    dev = _native.require_device(rows, cos, sin, k_cache, v_cache, lens, slot_ids, block_table)
    cr, sr = _rope_rows(cos, B, D), _rope_rows(sin, B, D)
    _require(cr.stride(0) == sr.stride(0), "cos and sin need the same row stride")
    lens, slot_ids, block_table = _index(lens), _index(slot_ids), _block_table(block_table)
    P = int(num_programs) if num_programs else default_decode_splits(B, H_kv, dev)
    _require(P >= 1, "num_programs must be >= 1")

    lib = _native.load()
    o = q_like
    if B == 0:
        return o
    if plan is not None:  # a step's plan (decode_plan with append=True)
        n_wg = _plan_workgroups(plan)
        partials, counters = _planned_buffers(lib, dev, B, H_q, H_kv, D, n_wg, counters)
        _native.check(
            lib.cie_paged_decode_qkv_rope_planned(
                o.data_ptr(), rows.data_ptr(), rows.stride(0), cr.data_ptr(), sr.data_ptr(),
                cr.stride(0), k_cache.data_ptr(), v_cache.data_ptr(), plan.data_ptr(),
                block_table.data_ptr(), partials.data_ptr(), counters.data_ptr(),
                B, H_q, H_kv, D, PAGE_SIZE, N_PAGES, k_cache.stride(0), k_cache.stride(1),
                block_table.stride(0), block_table.shape[1], n_wg,
                _native.ptr(err), _native.stream_handle(dev),
            ),
            "cie_paged_decode_qkv_rope_planned",
        )
        return o
    _require(P <= lib.cie_paged_decode_max_splits(), "num_programs above the kernel's split limit")
    partials, counters = _split_buffers(lib, dev, B, H_q, H_kv, D, P, counters)
    _native.check(
        lib.cie_paged_decode_qkv_rope(
            o.data_ptr(), rows.data_ptr(), rows.stride(0), cr.data_ptr(), sr.data_ptr(), cr.stride(0),
            k_cache.data_ptr(), v_cache.data_ptr(), lens.data_ptr(), slot_ids.data_ptr(),
            block_table.data_ptr(), partials.data_ptr(), counters.data_ptr(),
            B, H_q, H_kv, D, PAGE_SIZE, N_PAGES, k_cache.stride(0), k_cache.stride(1),
            block_table.stride(0), block_table.shape[1], lens.shape[0], P,
            _native.ptr(err), _native.stream_handle(dev),
        ),
        "cie_paged_decode_qkv_rope",
    )
    return o


def append_tokens_qkv_rope(qkv, cos, sin, k_cache, v_cache, pages, offsets, num_heads: int,
                           err=None):
    """Mixed-step QKV split + RoPE + ``KVStorage.mixed_update`` in one launch.

    Token t of ``qkv`` (1, T, (H_q + 2·H_kv)·D) is rotated with ``cos`` /
    ``sin`` row t; its k and v rows go to ``(pages[t], :, offsets[t])`` of the
    pools (kv_cache/storage.py:62-85) and the rotated q is returned as
    (1, T, H_q, D), ready for ``mixed_gqa_attention``.
    """
    N_PAGES, H_kv, PAGE_SIZE, D = k_cache.shape
    H_q = int(num_heads)
    rows = _qkv_rows(qkv, (H_q + 2 * H_kv) * D)
    T = rows.shape[0]
    q = rows.new_empty((1, T, H_q, D))
    _check_pool(q, k_cache, v_cache)
    _require(tuple(pages.shape) == (T,) and tuple(offsets.shape) == (T,), "pages / offsets must be (T,)")
    dev = _native.require_device(rows, cos, sin, k_cache, v_cache, pages, offsets)
    cr, sr = _rope_rows(cos, T, D), _rope_rows(sin, T, D)
    _require(cr.stride(0) == sr.stride(0), "cos and sin need the same row stride")
    pages, offsets = _index(pages), _index(offsets)
    lib = _native.load()
    _native.check(
        lib.cie_kv_append_tokens_qkv_rope(
            q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), rows.data_ptr(), rows.stride(0),
            cr.data_ptr(), sr.data_ptr(), cr.stride(0), pages.data_ptr(), offsets.data_ptr(),
            T, H_q, H_kv, PAGE_SIZE, D, N_PAGES, k_cache.stride(0), k_cache.stride(1),
            _native.ptr(err), _native.stream_handle(dev),
        ),
        "cie_kv_append_tokens_qkv_rope",
    )
    return q


def _as_rows(x: torch.Tensor, h_kv: int, d: int) -> torch.Tensor:
    try:
        rows = x.view(-1, h_kv, d)
    except RuntimeError:
        rows = x.reshape(-1, h_kv, d)
    if rows.stride(2) != 1 or rows.stride(0) % 8 or rows.stride(1) % 8 or rows.data_ptr() % 16:
        rows = rows.contiguous()
    return rows


def mixed_plan(k_cache, cu_seqlens, kv_lens, slot_ids, block_table, max_seqlen: int, total_T: int,
               num_heads: int, partials_bytes=None, err=None):
    """One mixed step's plan, made once and used by every layer's planned mixed attention.

    A mixed step's sequences (``cu_seqlens``, ``kv_lens`` = prior lengths,
    ``slot_ids``) are the same for every layer (the reference builds its
    ``AttentionMetadata`` once per step, attn/metadata.py:3-55): the plan holds
    the work items, their order and the partial bases that each launch of
    ``mixed_gqa_attention`` would otherwise work out for itself.  Pass it as
    ``plan=`` to the layers' calls with the same batch, ``total_T`` (q's
    packed rows), head count and ``partials_bytes``; the outputs are the
    unplanned ones bit for bit.  Returns an int32 device tensor.
    """
    N_PAGES, H_kv, PAGE_SIZE, D = k_cache.shape
    B = slot_ids.shape[0]
    _require(num_heads % H_kv == 0, "H_q must be a multiple of H_kv")
    _require(tuple(cu_seqlens.shape) == (B + 1,) and tuple(kv_lens.shape) == (B,),
             "cu_seqlens must be (B+1,) and kv_lens (B,)")
    _require(N_PAGES == block_table.shape[1], "block_table width must equal n_pages")
    dev = _native.require_device(k_cache, cu_seqlens, kv_lens, slot_ids, block_table)
    cu_seqlens, kv_lens, slot_ids = _index(cu_seqlens), _index(kv_lens), _index(slot_ids)
    lib = _native.load()
    n = lib.cie_mixed_plan_bytes(B, int(total_T))
    _require(n > 0, "batch too large for a mixed plan")
    plan = torch.empty(n // 4, dtype=torch.int32, device=dev)
    if partials_bytes is None:
        partials_bytes = lib.cie_mixed_partials_bytes(int(total_T), num_heads, D)
    _native.check(
        lib.cie_mixed_plan(
            plan.data_ptr(), n, cu_seqlens.data_ptr(), kv_lens.data_ptr(), slot_ids.data_ptr(), B,
            int(total_T), int(max_seqlen), num_heads, H_kv, D, PAGE_SIZE, block_table.shape[1],
            block_table.shape[0], partials_bytes, _native.ptr(err), _native.stream_handle(dev),
        ),
        "cie_mixed_plan",
    )
    return plan


def mixed_gqa_attention(q, k, v, max_seqlen: int, cu_seqlens, kv_lens, slot_ids, block_table,
                        BLOCK_M=16, BLOCK_N=64, num_warps=4, wrap=None, err=None, counters=None,
                        partials_bytes=None, plan=None):
    """Varlen causal GQA attention over the paged pool (chunked prefill + decode).

    q: (1, total_T, H_q, D) fp16 contiguous; cu_seqlens (B+1,); kv_lens (B,) =
    prior lengths; row i of sequence b attends keys [0, kv_lens[b] + i].
    Rows outside every sequence are left as ``torch.empty_like`` leaves them.
    ``partials_bytes`` is the budget of split-chunk partial state (default
    ``cie_mixed_partials_bytes``: per q head, the larger of 2 rows per token
    and 16 rows for each of the first 64 tokens, so the decode rows of a
    small batch can all split); sequences whose split tiles do not fit it
    run unsplit, with the same results.
    ``plan``: the step's ``mixed_plan`` (same batch, ``total_T``, heads and
    budget); ``cu_seqlens``, ``kv_lens`` and ``slot_ids`` are then read from it.
    """
    total_T, H_q, D = q.shape[1:]
    N_PAGES, H_kv, PAGE_SIZE, _ = k.shape
    B = slot_ids.shape[0]
    _require(H_q % H_kv == 0, "H_q must be a multiple of H_kv")
    _require(tuple(kv_lens.shape) == (B,), "kv_lens must be (B,)")
    _require(tuple(cu_seqlens.shape) == (B + 1,), "cu_seqlens must be (B+1,)")
    _require(N_PAGES == block_table.shape[1], "block_table width must equal n_pages")
    _require(q.is_contiguous() and k.is_contiguous() and v.is_contiguous(), "q, k, v must be contiguous")
    _check_pool(q, k, v)
    dev = _native.require_device(q, k, v, cu_seqlens, kv_lens, slot_ids, block_table)
    cu_seqlens, kv_lens, slot_ids = _index(cu_seqlens), _index(kv_lens), _index(slot_ids)
    block_table = _block_table(block_table)

    lib = _native.load()
    o = torch.empty_like(q)
    if B == 0 or total_T == 0 or int(max_seqlen) == 0:
        return o
    if partials_bytes is None:
        partials_bytes = lib.cie_mixed_partials_bytes(total_T, H_q, D)
    _require(partials_bytes >= 0, "partials_bytes must be >= 0")
    partials = torch.empty(partials_bytes, dtype=torch.uint8, device=dev)
    n_ctr = lib.cie_mixed_counters(B, H_kv, int(max_seqlen))
    if counters is None:
        counters = split_counters(dev, n_ctr)
    _require(counters.dtype == torch.int32 and counters.numel() >= n_ctr, "counters too small")
    if plan is not None:  # a step's plan (mixed_plan)
        n = lib.cie_mixed_plan_bytes(B, total_T)
        _require(plan.dtype == torch.int32 and plan.is_contiguous() and plan.numel() * 4 >= n,
                 "plan must come from mixed_plan for this batch")
        _native.check(
            lib.cie_mixed_attention_planned(
                o.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), plan.data_ptr(), plan.numel() * 4,
                block_table.data_ptr(),
                _native.ptr(partials) if partials_bytes else None, partials_bytes, counters.data_ptr(),
                B, total_T, int(max_seqlen), H_q, H_kv, D, PAGE_SIZE, N_PAGES,
                k.stride(0), k.stride(1), block_table.stride(0), block_table.shape[1],
                block_table.shape[0], _native.ptr(err), _native.stream_handle(dev),
            ),
            "cie_mixed_attention_planned",
        )
        return o
    _native.check(
        lib.cie_mixed_attention(
            o.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
            cu_seqlens.data_ptr(), kv_lens.data_ptr(), slot_ids.data_ptr(), block_table.data_ptr(),
            _native.ptr(partials) if partials_bytes else None, partials_bytes, counters.data_ptr(),
            B, total_T, int(max_seqlen), H_q, H_kv, D, PAGE_SIZE, N_PAGES,
            k.stride(0), k.stride(1), block_table.stride(0), block_table.shape[1],
            block_table.shape[0], _native.ptr(err), _native.stream_handle(dev),
        ),
        "cie_mixed_attention",
    )
    return o


# Op-level configs (the reference's GQA_DECODE_CONFIG / GQA_PREFILL_CONFIG,
# attn/core.py:114-116).  num_programs=None picks the split count per batch.
GQA_DECODE_CONFIG = {"num_programs": None}
GQA_PREFILL_CONFIG = {}


@torch.library.custom_op("inference::gqa_decode_attention", mutates_args=())
def gqa_decode_attention_op(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
    lens: torch.Tensor, slot_ids: torch.Tensor, block_table: torch.Tensor,
) -> torch.Tensor:
    return decode_gqa_attention(q, k, v, lens=lens, slot_ids=slot_ids, block_table=block_table,
                                **GQA_DECODE_CONFIG)


@gqa_decode_attention_op.register_fake
def _(q, k, v, lens, slot_ids, block_table):
    return torch.empty_like(q)


@torch.library.custom_op("inference::gqa_decode_append_attention", mutates_args=("k_cache", "v_cache"))
def gqa_decode_append_attention_op(
    q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, k: torch.Tensor,
    v: torch.Tensor, lens: torch.Tensor, slot_ids: torch.Tensor, block_table: torch.Tensor,
    plan: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    if plan is not None:
        return decode_append_gqa_attention(q, k_cache, v_cache, k, v, lens, slot_ids, block_table,
                                           plan=plan)
    return decode_append_gqa_attention(q, k_cache, v_cache, k, v, lens, slot_ids, block_table,
                                       **GQA_DECODE_CONFIG)


@gqa_decode_append_attention_op.register_fake
def _(q, k_cache, v_cache, k, v, lens, slot_ids, block_table, plan=None):
    return torch.empty_like(q)


@torch.library.custom_op("inference::gqa_decode_qkv_rope_attention",
                         mutates_args=("k_cache", "v_cache"))
def gqa_decode_qkv_rope_attention_op(
    qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, k_cache: torch.Tensor,
    v_cache: torch.Tensor, lens: torch.Tensor, slot_ids: torch.Tensor, block_table: torch.Tensor,
    num_heads: int, plan: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    if plan is not None:
        return decode_qkv_rope_gqa_attention(qkv, cos, sin, k_cache, v_cache, lens, slot_ids,
                                             block_table, num_heads, plan=plan)
    return decode_qkv_rope_gqa_attention(qkv, cos, sin, k_cache, v_cache, lens, slot_ids, block_table,
                                         num_heads, **GQA_DECODE_CONFIG)


@gqa_decode_qkv_rope_attention_op.register_fake
def _(qkv, cos, sin, k_cache, v_cache, lens, slot_ids, block_table, num_heads, plan=None):
    return qkv.new_empty((1, qkv.shape[1], num_heads, k_cache.shape[-1]))


@torch.library.custom_op("inference::gqa_decode_plan", mutates_args=())
def gqa_decode_plan_op(k_cache: torch.Tensor, lens: torch.Tensor, slot_ids: torch.Tensor,
                       block_table: torch.Tensor) -> torch.Tensor:
    """A decode step's plan for its fused-append layers (decode_plan, append=True)."""
    return decode_plan(k_cache, lens, slot_ids, block_table, append=True)


@gqa_decode_plan_op.register_fake
def _(k_cache, lens, slot_ids, block_table):
    n_wg = _native.load().cie_paged_decode_plan_workgroups(max(slot_ids.shape[0], 1), k_cache.shape[1], 0)
    return k_cache.new_empty((n_wg * PLAN_WORDS_PER_WORKGROUP,), dtype=torch.int32)


@torch.library.custom_op("inference::kv_append_tokens_qkv_rope", mutates_args=("k_cache", "v_cache"))
def kv_append_tokens_qkv_rope_op(
    qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, k_cache: torch.Tensor,
    v_cache: torch.Tensor, pages: torch.Tensor, offsets: torch.Tensor, num_heads: int,
) -> torch.Tensor:
    return append_tokens_qkv_rope(qkv, cos, sin, k_cache, v_cache, pages, offsets, num_heads)


@kv_append_tokens_qkv_rope_op.register_fake
def _(qkv, cos, sin, k_cache, v_cache, pages, offsets, num_heads):
    return qkv.new_empty((1, qkv.shape[1], num_heads, k_cache.shape[-1]))


@torch.library.custom_op("inference::gqa_mixed_attention", mutates_args=())
def gqa_mixed_attention_op(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
    max_seqlen: int, cu_seqlens: torch.Tensor, kv_lens: torch.Tensor,
    slot_ids: torch.Tensor, block_table: torch.Tensor, plan: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    return mixed_gqa_attention(q, k, v, **GQA_PREFILL_CONFIG, max_seqlen=max_seqlen,
                               cu_seqlens=cu_seqlens, block_table=block_table, kv_lens=kv_lens,
                               slot_ids=slot_ids, plan=plan)


@gqa_mixed_attention_op.register_fake
def _(q, k, v, max_seqlen, cu_seqlens, kv_lens, slot_ids, block_table, plan=None):
    return torch.empty_like(q)


@torch.library.custom_op("inference::gqa_mixed_plan", mutates_args=())
def gqa_mixed_plan_op(k_cache: torch.Tensor, cu_seqlens: torch.Tensor, kv_lens: torch.Tensor,
                      slot_ids: torch.Tensor, block_table: torch.Tensor, max_seqlen: int, total_T: int,
                      num_heads: int) -> torch.Tensor:
    """A mixed step's plan for its layers' mixed attention (mixed_plan)."""
    return mixed_plan(k_cache, cu_seqlens, kv_lens, slot_ids, block_table, max_seqlen, total_T, num_heads)


@gqa_mixed_plan_op.register_fake
def _(k_cache, cu_seqlens, kv_lens, slot_ids, block_table, max_seqlen, total_T, num_heads):
    n = _native.load().cie_mixed_plan_bytes(slot_ids.shape[0], total_T)
    return k_cache.new_empty((n // 4,), dtype=torch.int32)


class TritonQwen2Attention(torch.nn.Module):
    """Drop-in for HF ``Qwen2Attention`` over the paged pool (attn/core.py:139-236).

    Fused QKV projection -> RoPE -> KV append (decode or token mode) -> paged
    attention (decode or mixed) -> o_proj.  Falls back to the wrapped HF module
    when no ``kv_manager`` is passed.  By default the split, RoPE and append
    run inside the HIP kernels (``fuse_rope``; a decode step is one launch);
    ``fuse_rope = False`` / ``fuse_append = False`` select the reference's
    sequence of separate calls.
    """

    def __init__(self, original_attn):
        super().__init__()
        if original_attn.sliding_window is not None:
            raise AssertionError("sliding window attention is not supported")
        self.original = original_attn
        self.layer_idx = original_attn.layer_idx
        self.num_heads = original_attn.config.num_attention_heads
        self.head_dim = original_attn.head_dim
        if original_attn.scaling != self.head_dim ** -0.5:
            raise AssertionError("only the default 1/sqrt(head_dim) scaling is supported")
        projs = [original_attn.q_proj, original_attn.k_proj, original_attn.v_proj]
        if not all(p.bias is not None for p in projs):
            raise AssertionError("q/k/v projections must have biases")
        self.qkv_sizes = [p.out_features for p in projs]
        with torch.no_grad():
            self.register_buffer("qkv_weight", torch.cat([p.weight for p in projs]), persistent=False)
            self.register_buffer("qkv_bias", torch.cat([p.bias for p in projs]), persistent=False)
        self.fuse_qkv = True
        # decode branch: KV append fused into the decode launch (one kernel)
        # instead of decode_update + gqa_decode_attention (two).
        self.fuse_append = True
        # QKV split + RoPE fused into the append kernels (decode: into the
        # decode launch; mixed: one append launch that also emits rotated q)
        # instead of views, apply_rotary_pos_emb's elementwise kernels and the
        # plain append.
        self.fuse_rope = True

    def forward(self, hidden_states, position_embeddings, attention_mask=None,
                past_key_values=None, kv_manager=None, **kwargs):
        if kv_manager is None:
            return self.original(hidden_states, position_embeddings, attention_mask,
                                 past_key_values=past_key_values, **kwargs)
        metadata = kwargs.get("metadata")
        if metadata is None:
            raise ValueError("'metadata' is required with custom kv_manager.")

        attn = self.original
        total_T = hidden_states.shape[1]
        hidden_shape = (1, total_T, -1, self.head_dim)
        keys, values = kv_manager.keys[self.layer_idx], kv_manager.values[self.layer_idx]
        if self.fuse_qkv and self.fuse_rope and (self.fuse_append or not metadata.full_decode):
            qkv = torch.nn.functional.linear(hidden_states, self.qkv_weight, self.qkv_bias)
            cos, sin = position_embeddings
            if metadata.full_decode:
                o = gqa_decode_qkv_rope_attention_op(
                    qkv, cos, sin, keys, values, kv_manager.lens, metadata.slot_ids,
                    kv_manager.block_table, self.num_heads, plan=getattr(metadata, "decode_plan", None),
                )
            else:
                query_states = kv_append_tokens_qkv_rope_op(
                    qkv, cos, sin, keys, values, metadata.pages, metadata.offsets, self.num_heads,
                )
                o = gqa_mixed_attention_op(
                    query_states, keys, values,
                    kv_lens=kv_manager.lens[metadata.slot_ids], max_seqlen=metadata.max_seqlen,
                    cu_seqlens=metadata.cu_seqlens, slot_ids=metadata.slot_ids,
                    block_table=kv_manager.block_table, plan=getattr(metadata, "mixed_plan", None),
                )
            attn_output = attn.o_proj(o.reshape(1, total_T, self.num_heads * self.head_dim))
            return attn_output, None

        if self.fuse_qkv:
            q, k, v = torch.nn.functional.linear(hidden_states, self.qkv_weight, self.qkv_bias).split(
                self.qkv_sizes, dim=-1)
        else:
            q, k, v = attn.q_proj(hidden_states), attn.k_proj(hidden_states), attn.v_proj(hidden_states)
        query_states = q.view(hidden_shape)
        key_states = k.view(hidden_shape)
        value_states = v.view(hidden_shape)
        cos, sin = position_embeddings
        query_states, key_states = apply_rotary_pos_emb(query_states, key_states, cos, sin,
                                                        unsqueeze_dim=2)

        if metadata.full_decode and self.fuse_append:
            o = gqa_decode_append_attention_op(
                query_states, kv_manager.keys[self.layer_idx], kv_manager.values[self.layer_idx],
                key_states, value_states, kv_manager.lens, metadata.slot_ids, kv_manager.block_table,
                plan=getattr(metadata, "decode_plan", None),
            )
        elif metadata.full_decode:
            kv_manager.decode_update(self.layer_idx, metadata.slot_ids, key_states, value_states)
            o = gqa_decode_attention_op(
                query_states, kv_manager.keys[self.layer_idx], kv_manager.values[self.layer_idx],
                kv_manager.lens[metadata.slot_ids] + 1,
                slot_ids=metadata.slot_ids, block_table=kv_manager.block_table,
            )
        else:
            kv_manager.mixed_update(self.layer_idx, metadata.pages, metadata.offsets,
                                    key_states, value_states)
            o = gqa_mixed_attention_op(
                query_states, kv_manager.keys[self.layer_idx], kv_manager.values[self.layer_idx],
                kv_lens=kv_manager.lens[metadata.slot_ids], max_seqlen=metadata.max_seqlen,
                cu_seqlens=metadata.cu_seqlens, slot_ids=metadata.slot_ids,
                block_table=kv_manager.block_table, plan=getattr(metadata, "mixed_plan", None),
            )
        attn_output = attn.o_proj(o.reshape(1, total_T, self.num_heads * self.head_dim))
        return attn_output, None


HipQwen2Attention = TritonQwen2Attention


def replace_attention(module) -> None:
    for name, child in module.named_children():
        if isinstance(child, Qwen2Attention):
            setattr(module, name, TritonQwen2Attention(child))
        elif not isinstance(child, TritonQwen2Attention):
            replace_attention(child)


def use_triton_attention(model) -> None:
    if not getattr(model, "_uses_triton_attention", False):
        replace_attention(model)
        model._uses_triton_attention = True
