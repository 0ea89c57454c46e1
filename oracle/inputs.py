"""Seeded synthetic inputs for the BASELINE configurations (test / bench infrastructure).

TEST INFRASTRUCTURE ONLY (see oracle/paged_attention.py).  The reference ships
no input recipe, so this one is the build's, fixed here:

  one ``torch.Generator("cpu").manual_seed(seed)`` per case, drawn in order
    1. random prior lengths, when the config asks for them (torch.randint);
    2. the page assignment: ``randperm(n_pages - 1) + 1`` cut into consecutive
       per-sequence runs (page 0 never handed out, as KVStorage reserves it,
       kv_cache/storage.py:20);
    3. the whole K pool, then the whole V pool, ``randn * 0.5`` -> fp16
       (so a read of a wrong page shows up as an error);
    4. new k, then new v, ``(1, T, H_kv, D)``;
    5. q ``(1, T, H_q, D)``.
  Slot 0 is the reserved padding slot; sequences use slots 1..B.  The block
  table is (n_slots, bt_width) int64 with unused entries 0; bt_width defaults
  to n_pages, as the reference requires (attn/core.py:20).  Pools are sized to
  fit, ``1 + sum(ceil((prior + new) / page_size))`` pages, unless given.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import paged_attention as ref


@dataclass
class PagedCase:
    q: torch.Tensor            # (1, T, H_q, D) fp16
    k_new: torch.Tensor        # (1, T, H_kv, D) fp16
    v_new: torch.Tensor
    k_pool: torch.Tensor       # (n_pages, H_kv, P, D) fp16, before the append
    v_pool: torch.Tensor
    block_table: torch.Tensor  # (n_slots, bt_width) int64
    lens_pool: torch.Tensor    # (n_slots,) int64 prior lengths per slot
    slot_ids: torch.Tensor     # (B,) int64
    kv_lens: torch.Tensor      # (B,) int64 prior lengths
    new_lens: torch.Tensor     # (B,) int64 query rows per sequence
    cu_seqlens: torch.Tensor   # (B+1,) int64
    pages: torch.Tensor        # (T,) int64 append page per token
    offsets: torch.Tensor      # (T,) int64 append offset per token
    page_size: int
    meta: dict = field(default_factory=dict)

    @property
    def B(self) -> int:
        return int(self.slot_ids.shape[0])

    @property
    def T(self) -> int:
        return int(self.q.shape[1])

    @property
    def attended(self) -> torch.Tensor:
        """Decode attended length per sequence (prior + the appended token)."""
        return self.kv_lens + self.new_lens

    def appended_pools(self) -> tuple[torch.Tensor, torch.Tensor]:
        """Pools after the token-mode append of every new row (oracle)."""
        kp, vp = self.k_pool.clone(), self.v_pool.clone()
        ref.append_tokens(kp, vp, self.k_new, self.v_new, self.pages, self.offsets)
        return kp, vp

    def to(self, device) -> "PagedCase":
        moved = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in self.__dict__.items()}
        return PagedCase(**moved)


def make_case(prior_lens, new_lens=None, *, h_q=14, h_kv=2, d=64, page_size=16, n_pages=None,
              bt_width=None, seed=0, random_lens=None, n_slots=None,
              full_row: bool = False) -> PagedCase:
    """Build one seeded case.

    prior_lens: list of prior KV lengths (ignored when random_lens=(lo, hi, B)
    draws them uniformly in [lo, hi]).  new_lens: query rows per sequence
    (default 1 each: a decode step).  full_row (B == 1 only): the sequence's
    block-table row holds the whole permutation of pages 1..n_pages-1.
    """
    g = torch.Generator("cpu").manual_seed(seed)
    if random_lens is not None:
        lo, hi, nb = random_lens
        prior = torch.randint(lo, hi + 1, (nb,), generator=g).tolist()
    else:
        prior = [int(x) for x in prior_lens]
    B = len(prior)
    new = [1] * B if new_lens is None else [int(x) for x in new_lens]
    assert len(new) == B
    need = [-(-(c + n) // page_size) for c, n in zip(prior, new)]
    if n_pages is None:
        n_pages = 1 + sum(need)
    assert 1 + sum(need) <= n_pages, "pool too small for the case"
    if bt_width is None:
        bt_width = n_pages
    assert max(need, default=0) <= bt_width
    n_slots = n_slots or B + 1

    perm = torch.randperm(n_pages - 1, generator=g) + 1
    block_table = torch.zeros(n_slots, bt_width, dtype=torch.int64)
    if full_row:
        assert B == 1 and bt_width >= n_pages - 1
        block_table[1, :n_pages - 1] = perm
    else:
        at = 0
        for i, n in enumerate(need):
            block_table[1 + i, :n] = perm[at:at + n]
            at += n
    k_pool = (torch.randn(n_pages, h_kv, page_size, d, generator=g) * 0.5).half()
    v_pool = (torch.randn(n_pages, h_kv, page_size, d, generator=g) * 0.5).half()
    T = sum(new)
    k_new = (torch.randn(1, T, h_kv, d, generator=g) * 0.5).half()
    v_new = (torch.randn(1, T, h_kv, d, generator=g) * 0.5).half()
    q = (torch.randn(1, T, h_q, d, generator=g) * 0.5).half()

    slot_ids = torch.arange(1, B + 1, dtype=torch.int64)
    lens_pool = torch.zeros(n_slots, dtype=torch.int64)
    lens_pool[1:B + 1] = torch.tensor(prior, dtype=torch.int64)
    new_t = torch.tensor(new, dtype=torch.int64)
    cu = torch.zeros(B + 1, dtype=torch.int64)
    cu[1:] = torch.cumsum(new_t, 0)
    pages, offsets, _ = ref.mixed_pages_offsets(lens_pool, block_table, slot_ids, cu, page_size)
    return PagedCase(q=q, k_new=k_new, v_new=v_new, k_pool=k_pool, v_pool=v_pool,
                     block_table=block_table, lens_pool=lens_pool, slot_ids=slot_ids,
                     kv_lens=torch.tensor(prior, dtype=torch.int64), new_lens=new_t,
                     cu_seqlens=cu, pages=pages, offsets=offsets, page_size=page_size,
                     meta={"seed": seed, "n_pages": n_pages})


# BASELINE.json configs -------------------------------------------------------

def config1(seed: int = 0) -> PagedCase:
    """B=1, kv_len 128, 64-page pool; block-table row = randperm(63) + 1 (all 63 pages)."""
    case = make_case([128], n_pages=64, seed=seed, full_row=True)
    case.meta["n_splits"] = 4
    return case


def config2(seed: int = 0, fixed: bool = True) -> PagedCase:
    """B=32 decode; prior 4096 each (headline) or U[512, 4096]."""
    if fixed:
        return make_case([4096] * 32, seed=seed)
    return make_case(None, random_lens=(512, 4096, 32), seed=seed)


def config3(seed: int = 0) -> PagedCase:
    """4 prefill chunks of 256 rows (prior 0, 512, 1024, 2048) + 28 decode rows (prior U[256, 3072])."""
    g = torch.Generator("cpu").manual_seed(seed + 20_000)
    dec = torch.randint(256, 3073, (28,), generator=g).tolist()
    prior = [0, 512, 1024, 2048] + dec
    new = [256] * 4 + [1] * 28
    case = make_case(prior, new, seed=seed)
    case.meta["max_seqlen"] = 256
    return case


def config4(seed: int = 0) -> PagedCase:
    """B=16, prior 16384 each (attend 16385), 16 splits."""
    case = make_case([16384] * 16, seed=seed)
    case.meta["n_splits"] = 16
    return case
