"""Paged KV pool with the reference's ``KVStorage`` surface.

Mirrors kv_cache/storage.py:4-141 of the reference: per-layer pools of shape
``(n_pages, H_kv, page_size, D)``, ``lens (n_slots,)``, ``block_table
(n_slots, n_pages)`` and ``last_generated (n_slots,)``, with slot 0 and page 0
reserved as the padding target (``unused_idx = 0``).  The two appends run the
gfx950 ``kv_append`` kernel through the ``inference::kv_append_decode`` /
``inference::kv_append_tokens`` custom ops (declared as mutating the pools, so
``torch.compile`` keeps them in order), instead of torch gathers plus
``index_put_``.

All layers' K (and V) pages live in one allocation ``(num_layers, n_pages,
H_kv, page_size, D)``; ``keys[l]`` / ``values[l]`` are dense per-layer views,
so the per-layer tensors have exactly the reference's shape and strides.
"""
from __future__ import annotations

import math

import torch

from .. import _native


def _as_rows(x: torch.Tensor, h_kv: int, d: int) -> torch.Tensor:
    # The reference views the new K/V as (-1, H_kv, D) (storage.py:75, 83, 110, 122);
    # a strided view (V straight out of the fused QKV split) keeps its strides.
    try:
        rows = x.view(-1, h_kv, d)
    except RuntimeError:
        rows = x.reshape(-1, h_kv, d)
    if rows.stride(2) != 1:
        rows = rows.contiguous()
    return rows


def _index(t: torch.Tensor) -> torch.Tensor:
    if t.dtype != torch.int64 or not t.is_contiguous():
        t = t.to(torch.int64).contiguous()
    return t


def _check_pools(k_cache: torch.Tensor, v_cache: torch.Tensor) -> None:
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape:
        raise AssertionError("K/V pools must both be (n_pages, H_kv, page_size, D)")
    if k_cache.stride() != v_cache.stride() or k_cache.stride(3) != 1 or k_cache.stride(2) != k_cache.shape[3]:
        raise AssertionError("K/V pools need identical strides with dense (page_size, D) rows")
    if k_cache.element_size() != 2 or v_cache.dtype != k_cache.dtype:
        raise AssertionError("K/V pools must share a 2-byte dtype")


def kv_append_decode(k_cache, v_cache, k, v, slot_ids, lens, block_table, err=None) -> None:
    """``K[block_table[s, lens[s] // P], :, lens[s] % P] = k[b]`` for s = slot_ids[b] (same for V).

    Follows KVStorage.decode_update (kv_cache/storage.py:87-122); one launch
    writes both pools.  ``lens`` is the pool's per-slot length (n_slots,).
    """
    _check_pools(k_cache, v_cache)
    n_pages, h_kv, page_size, d = k_cache.shape
    dev = _native.require_device(k_cache, v_cache, k, v, slot_ids, lens, block_table)
    kr, vr = _as_rows(k, h_kv, d), _as_rows(v, h_kv, d)
    if kr.dtype != k_cache.dtype or vr.dtype != k_cache.dtype:
        raise AssertionError("new K/V dtype must match the pool")
    slot_ids, lens, block_table = _index(slot_ids), _index(lens), block_table
    if block_table.dtype != torch.int64 or block_table.stride(1) != 1:
        block_table = block_table.to(torch.int64).contiguous()
    B = slot_ids.shape[0]
    if kr.shape[0] != B or vr.shape[0] != B:
        raise AssertionError(f"expected {B} new rows, got {kr.shape[0]} / {vr.shape[0]}")
    lib = _native.load()
    _native.check(
        lib.cie_kv_append_decode(
            k_cache.data_ptr(), v_cache.data_ptr(), kr.data_ptr(), vr.data_ptr(),
            kr.stride(0), kr.stride(1), vr.stride(0), vr.stride(1),
            slot_ids.data_ptr(), lens.data_ptr(), block_table.data_ptr(),
            B, h_kv, page_size, d, n_pages, k_cache.stride(0), k_cache.stride(1),
            block_table.stride(0), block_table.shape[1], lens.shape[0],
            _native.ptr(err), _native.stream_handle(dev),
        ),
        "cie_kv_append_decode",
    )


def kv_append_tokens(k_cache, v_cache, k, v, pages, offsets, err=None) -> None:
    """``K[pages[t], :, offsets[t]] = k[t]`` for every packed token (same for V).

    Follows KVStorage.mixed_update (kv_cache/storage.py:62-85).
    """
    _check_pools(k_cache, v_cache)
    n_pages, h_kv, page_size, d = k_cache.shape
    dev = _native.require_device(k_cache, v_cache, k, v, pages, offsets)
    kr, vr = _as_rows(k, h_kv, d), _as_rows(v, h_kv, d)
    if kr.dtype != k_cache.dtype or vr.dtype != k_cache.dtype:
        raise AssertionError("new K/V dtype must match the pool")
    pages, offsets = _index(pages), _index(offsets)
    T = pages.shape[0]
    if offsets.shape[0] != T or kr.shape[0] != T or vr.shape[0] != T:
        raise AssertionError("pages, offsets and new K/V must have one row per token")
    lib = _native.load()
    _native.check(
        lib.cie_kv_append_tokens(
            k_cache.data_ptr(), v_cache.data_ptr(), kr.data_ptr(), vr.data_ptr(),
            kr.stride(0), kr.stride(1), vr.stride(0), vr.stride(1),
            pages.data_ptr(), offsets.data_ptr(), T, h_kv, page_size, d, n_pages,
            k_cache.stride(0), k_cache.stride(1), _native.ptr(err), _native.stream_handle(dev),
        ),
        "cie_kv_append_tokens",
    )


@torch.library.custom_op("inference::kv_append_decode", mutates_args=("k_cache", "v_cache"))
def kv_append_decode_op(
    k_cache: torch.Tensor, v_cache: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
    slot_ids: torch.Tensor, lens: torch.Tensor, block_table: torch.Tensor,
) -> None:
    kv_append_decode(k_cache, v_cache, k, v, slot_ids, lens, block_table)


@kv_append_decode_op.register_fake
def _(k_cache, v_cache, k, v, slot_ids, lens, block_table) -> None:
    return None


@torch.library.custom_op("inference::kv_append_tokens", mutates_args=("k_cache", "v_cache"))
def kv_append_tokens_op(
    k_cache: torch.Tensor, v_cache: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
    pages: torch.Tensor, offsets: torch.Tensor,
) -> None:
    kv_append_tokens(k_cache, v_cache, k, v, pages, offsets)


@kv_append_tokens_op.register_fake
def _(k_cache, v_cache, k, v, pages, offsets) -> None:
    return None


class KVStorage:
    """Paged per-layer K/V pools plus per-slot lengths and block tables.

    Same constructor and attributes as the reference (kv_cache/storage.py:6-60).
    """

    def __init__(self, config, max_cache_len, page_size, n_slots, device, dtype):
        self.config = config
        self.max_cache_len = max_cache_len
        self.page_size = page_size
        self.n_slots = n_slots
        self.device = device
        self.dtype = dtype

        self.n_pages = math.ceil(max_cache_len / page_size)
        self.unused_idx = 0

        self.num_layers = config.num_hidden_layers
        self.num_q_heads = config.num_attention_heads
        self.num_kv_heads = config.num_key_value_heads
        self.head_dim = getattr(config, "head_dim", None) or config.hidden_size // config.num_attention_heads

        shape = (self.num_layers, self.n_pages, self.num_kv_heads, self.page_size, self.head_dim)
        self._k_storage = torch.zeros(shape, device=device, dtype=dtype)
        self._v_storage = torch.zeros(shape, device=device, dtype=dtype)
        self.keys = list(self._k_storage.unbind(0))
        self.values = list(self._v_storage.unbind(0))

        self.lens = torch.zeros((n_slots,), dtype=torch.long, device=self.device)
        self.block_table = torch.zeros((n_slots, self.n_pages), dtype=torch.long, device=self.device)
        self.last_generated = torch.zeros((n_slots,), dtype=torch.long, device=self.device)

    def mixed_update(self, layer_num: int, pages: torch.Tensor, offsets: torch.Tensor,
                     k_proj: torch.Tensor, v_proj: torch.Tensor) -> None:
        torch.ops.inference.kv_append_tokens(
            self.keys[layer_num], self.values[layer_num], k_proj, v_proj, pages, offsets
        )

    def decode_update(self, layer_num: int, slot_ids: torch.Tensor,
                      k_proj: torch.Tensor, v_proj: torch.Tensor) -> None:
        torch.ops.inference.kv_append_decode(
            self.keys[layer_num], self.values[layer_num], k_proj, v_proj,
            slot_ids, self.lens, self.block_table,
        )

    # lens[unused_idx] = 0 as a device kernel (a 1-element multiply), not a
    # host scalar copy, so a decode step that contains it can be graph-captured
    # (and no memset node lands in the graph).
    def decode_advance(self, slot_ids: torch.Tensor) -> None:
        self.lens[slot_ids] += 1
        self.lens[self.unused_idx:self.unused_idx + 1].mul_(0)

    def mixed_advance(self, slot_ids: torch.Tensor, lens: torch.Tensor) -> None:
        self.lens[slot_ids] += lens
        self.lens[self.unused_idx:self.unused_idx + 1].mul_(0)

    def reset(self, slot_ids: list[int]) -> None:
        self.lens[slot_ids] = 0
        self.block_table[slot_ids] = 0
