"""CPU oracle for the paged-KV GQA attention hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this module, and only as the
checker (or, in bench.py, as the timed CPU baseline) — never as a product code
path.  The product (``custom_inference_engine_amd``) has no CPU fallback.

Each function restates the reference's semantics (file:line under the
reference repository) in plain numpy (byte / index work) or fp32 torch on the
CPU (attention arithmetic):

  append_decode            kv_cache/storage.py:87-122   (KVStorage.decode_update)
  append_tokens            kv_cache/storage.py:62-85    (KVStorage.mixed_update)
  decode_attention         attn/core.py:13-66 + kernels/decode_attention.py:12-272
                           as the exact softmax the split kernels compute
  decode_attention_splitkv kernels/decode_attention.py:71-141 (interleaved splits,
                           fp16 P) + :243-264 (log-sum-exp merge, -inf guard)
  mixed_attention          attn/core.py:69-111 + kernels/prefill_attention.py:37-198
  rope                     attn/core.py:193-198 (transformers' apply_rotary_pos_emb),
                           in fp32, rounded once to fp16
  *_bruteforce             scalar Python loops of the same definitions (tiny inputs)

Pins (tests/test_oracle.py): brute-force loops, torch's
``scaled_dot_product_attention`` (a library routine) on contiguous K/V, closed
forms (single key -> v0, equal keys -> mean of V, empty -> 0), invariants (page
permutation, split count, L=1 mixed == decode), and planted mistakes that the
pins must catch.  ``rope`` is pinned against transformers'
``apply_rotary_pos_emb`` run in fp32 (a library routine), the identity at
angle 0 and the 2-D rotation closed form.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F


# ----------------------------------------------------------------------------- rope

def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x*cos + rotate_half(x)*sin of apply_rotary_pos_emb (attn/core.py:193-198).

    x (T, H, D) fp16; cos / sin (T, D) fp16 (the rotary tables of each token's
    position); rotate_half(x) = cat(-x[..., D/2:], x[..., :D/2]).  The products
    of fp16 values are exact in fp32, so computing in fp32 rounds each output
    once (then to fp16) — what a fused fp32 kernel (or torch.compile's) stores.
    """
    xf = x.float()
    c, s = cos.float()[:, None, :], sin.float()[:, None, :]
    half = xf.shape[-1] // 2
    rot = torch.cat([-xf[..., half:], xf[..., :half]], dim=-1)
    return (xf * c + rot * s).half()


# ----------------------------------------------------------------------------- append

def append_decode(k_pool: torch.Tensor, v_pool: torch.Tensor, k_new: torch.Tensor,
                  v_new: torch.Tensor, slot_ids: torch.Tensor, lens: torch.Tensor,
                  block_table: torch.Tensor) -> None:
    """In place: pool[block_table[s, lens[s] // P], :, lens[s] % P] = new[b] (kv_cache/storage.py:95-122).

    ``lens`` is the pool's per-slot prior length (n_slots,).  numpy advanced
    indexing places the (B,) index dimension first, exactly as torch does for
    ``k_cache[pages, :, starts]``, so the value is (B, H_kv, D).
    """
    kp, vp = k_pool.numpy(), v_pool.numpy()
    _, h_kv, page_size, d = kp.shape
    slots = slot_ids.numpy()
    pos = lens.numpy()[slots]
    pages = block_table.numpy()[slots, pos // page_size]
    offs = pos % page_size
    kp[pages, :, offs] = k_new.numpy().reshape(-1, h_kv, d)
    vp[pages, :, offs] = v_new.numpy().reshape(-1, h_kv, d)


def append_tokens(k_pool: torch.Tensor, v_pool: torch.Tensor, k_new: torch.Tensor,
                  v_new: torch.Tensor, pages: torch.Tensor, offsets: torch.Tensor) -> None:
    """In place: pool[pages[t], :, offsets[t]] = new[t] (kv_cache/storage.py:75-83)."""
    kp, vp = k_pool.numpy(), v_pool.numpy()
    _, h_kv, _, d = kp.shape
    pg, off = pages.numpy(), offsets.numpy()
    kp[pg, :, off] = k_new.numpy().reshape(-1, h_kv, d)
    vp[pg, :, off] = v_new.numpy().reshape(-1, h_kv, d)


def append_decode_bruteforce(k_pool, v_pool, k_new, v_new, slot_ids, lens, block_table) -> None:
    """Scalar-loop statement of append_decode (one row copy at a time)."""
    _, h_kv, page_size, d = k_pool.shape
    kn = k_new.reshape(-1, h_kv, d)
    vn = v_new.reshape(-1, h_kv, d)
    for b in range(slot_ids.shape[0]):
        s = int(slot_ids[b])
        pos = int(lens[s])
        page = int(block_table[s, pos // page_size])
        for h in range(h_kv):
            k_pool[page, h, pos % page_size, :] = kn[b, h]
            v_pool[page, h, pos % page_size, :] = vn[b, h]


def mixed_pages_offsets(lens_pool: torch.Tensor, block_table: torch.Tensor,
                        slot_ids: torch.Tensor, cu_seqlens: torch.Tensor,
                        page_size: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Per-token (pages, offsets, positions) of a packed batch.

    scheduler/mixed_module.py:99-132: extended_slot_ids = repeat(slot_ids, L),
    pos = lens[slot] + offset_in_chunk, pages = block_table[slot, pos // P],
    offsets = pos % P.
    """
    cu = cu_seqlens.numpy()
    L = np.diff(cu)
    ext = np.repeat(slot_ids.numpy(), L)
    within = np.arange(int(cu[-1])) - np.repeat(cu[:-1], L)
    pos = lens_pool.numpy()[ext] + within
    pages = block_table.numpy()[ext, pos // page_size]
    return (torch.from_numpy(pages.astype(np.int64)), torch.from_numpy((pos % page_size).astype(np.int64)),
            torch.from_numpy(pos.astype(np.int64)))


# ----------------------------------------------------------------------------- gathers

def gather_seq(pool: torch.Tensor, block_table: torch.Tensor, slot: int, n: int) -> torch.Tensor:
    """First n tokens of a slot as (H_kv, n, D) fp32 (kernels/decode_attention.py:78-111)."""
    _, h_kv, page_size, d = pool.shape
    n_pg = -(-n // page_size)
    idx = block_table[slot, :n_pg]
    return pool[idx].float().permute(1, 0, 2, 3).reshape(h_kv, n_pg * page_size, d)[:, :n]


# ----------------------------------------------------------------------------- decode

def decode_attention(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                     lens: torch.Tensor, slot_ids: torch.Tensor,
                     block_table: torch.Tensor) -> torch.Tensor:
    """Exact fp32 paged GQA decode: (1, B, H_q, D) fp16 q -> (B, H_q, D) fp32.

    For each sequence b: gather lens[b] tokens of slot slot_ids[b], expand kv
    head g to its G = H_q / H_kv query heads (h // G), softmax(q K^T / sqrt(D)) V;
    lens[b] == 0 gives 0 (kernels/decode_attention.py:260-264).
    """
    _, B, h_q, d = q.shape
    h_kv = k_pool.shape[1]
    G = h_q // h_kv
    out = torch.zeros(B, h_q, d, dtype=torch.float32)
    for b in range(B):
        L = int(lens[b])
        if L == 0:
            continue
        s = int(slot_ids[b])
        K = gather_seq(k_pool, block_table, s, L).repeat_interleave(G, dim=0)
        V = gather_seq(v_pool, block_table, s, L).repeat_interleave(G, dim=0)
        qb = q[0, b].float().view(1, h_q, 1, d)
        out[b] = F.scaled_dot_product_attention(qb, K[None], V[None])[0, :, 0]
    return out


def decode_attention_bruteforce(q, k_pool, v_pool, lens, slot_ids, block_table) -> torch.Tensor:
    """Scalar loops: for every (b, h) walk tokens j < lens[b] through the block table."""
    _, B, h_q, d = q.shape
    _, h_kv, page_size, _ = k_pool.shape
    G = h_q // h_kv
    qf, kf, vf = q.double().numpy(), k_pool.double().numpy(), v_pool.double().numpy()
    bt = block_table.numpy()
    out = np.zeros((B, h_q, d))
    scale = 1.0 / math.sqrt(d)
    for b in range(B):
        s, L = int(slot_ids[b]), int(lens[b])
        for h in range(h_q):
            g = h // G
            scores = []
            for j in range(L):
                page, off = bt[s, j // page_size], j % page_size
                scores.append(sum(qf[0, b, h, x] * kf[page, g, off, x] for x in range(d)) * scale)
            if not scores:
                continue
            m = max(scores)
            w = [math.exp(sc - m) for sc in scores]
            tot = sum(w)
            for j in range(L):
                page, off = bt[s, j // page_size], j % page_size
                out[b, h] += (w[j] / tot) * vf[page, g, off]
    return torch.from_numpy(out).float()


def decode_attention_splitkv(q, k_pool, v_pool, lens, slot_ids, block_table,
                             num_programs: int, block_n: int = 16) -> torch.Tensor:
    """The reference's split-KV algorithm, step for step, in fp32 torch.

    Program p of P walks row blocks start = p*BN, p*BN + P*BN, ... below L
    (kernels/decode_attention.py:71-75); per block: s = (q.K^T) * D^-0.5 with
    rows >= L at -inf (:114-125), m_new = max(m_old, rowmax), p = exp(s - m_new),
    l = l*alpha + sum(p), acc = acc*alpha + fp16(p) . V (:127-141).  The merge
    (:243-264) forms sum_p e^(m_p-M) acc_p / sum_p e^(m_p-M) l_p, and 0 when
    every m_p is -inf.
    """
    _, B, h_q, d = q.shape
    h_kv = k_pool.shape[1]
    G = h_q // h_kv
    P = num_programs
    out = torch.zeros(B, h_q, d)
    for b in range(B):
        L, s = int(lens[b]), int(slot_ids[b])
        K = gather_seq(k_pool, block_table, s, L).repeat_interleave(G, dim=0) if L else None
        V = gather_seq(v_pool, block_table, s, L).repeat_interleave(G, dim=0) if L else None
        qb = q[0, b].float()
        pm = torch.full((P, h_q), -math.inf)
        pl = torch.zeros(P, h_q)
        pacc = torch.zeros(P, h_q, d)
        for p in range(P):
            m = torch.full((h_q,), -math.inf)
            l = torch.zeros(h_q)
            acc = torch.zeros(h_q, d)
            for start in range(p * block_n, L, P * block_n):
                stop = min(start + block_n, L)
                sc = torch.einsum("hd,hnd->hn", qb, K[:, start:stop]) * d ** -0.5
                m_new = torch.maximum(m, sc.max(dim=1).values)
                pe = torch.exp(sc - m_new[:, None])
                alpha = torch.exp(m - m_new)
                l = l * alpha + pe.sum(dim=1)
                acc = acc * alpha[:, None] + torch.einsum(
                    "hn,hnd->hd", pe.half().float(), V[:, start:stop])
                m = m_new
            pm[p], pl[p], pacc[p] = m, l, acc
        M = pm.max(dim=0).values
        alive = M > -math.inf
        a = torch.where(alive[None], torch.exp(pm - torch.where(alive, M, 0.0)[None]), 0.0)
        num = (pacc * a[..., None]).sum(0)
        den = (pl * a).sum(0)
        out[b] = torch.where(alive[:, None], num / torch.where(den > 0, den, 1.0)[:, None], 0.0)
    return out


# ----------------------------------------------------------------------------- mixed

def mixed_attention(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                    cu_seqlens: torch.Tensor, kv_lens: torch.Tensor, slot_ids: torch.Tensor,
                    block_table: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Exact fp32 varlen causal GQA attention -> ((T, H_q, D) fp32, written-row mask (T,)).

    Sequence b owns rows [cu[b], cu[b+1]); row i attends keys j <= kv_lens[b] + i
    of slot slot_ids[b] (kernels/prefill_attention.py:87, 145-146).  Rows outside
    every sequence are not written (the reference leaves empty_like garbage).
    """
    _, T, h_q, d = q.shape
    h_kv = k_pool.shape[1]
    G = h_q // h_kv
    out = torch.zeros(T, h_q, d)
    written = torch.zeros(T, dtype=torch.bool)
    cu = cu_seqlens.tolist()
    for b in range(slot_ids.shape[0]):
        t0, t1 = cu[b], cu[b + 1]
        L = t1 - t0
        if L <= 0:
            continue
        c, s = int(kv_lens[b]), int(slot_ids[b])
        E = c + L
        K = gather_seq(k_pool, block_table, s, E).repeat_interleave(G, dim=0)
        V = gather_seq(v_pool, block_table, s, E).repeat_interleave(G, dim=0)
        Q = q[0, t0:t1].float().permute(1, 0, 2)  # (H_q, L, D)
        allow = torch.arange(E)[None, :] <= (c + torch.arange(L))[:, None]
        o = F.scaled_dot_product_attention(Q[None], K[None], V[None], attn_mask=allow)
        out[t0:t1] = o[0].permute(1, 0, 2)
        written[t0:t1] = True
    return out, written


def mixed_attention_bruteforce(q, k_pool, v_pool, cu_seqlens, kv_lens, slot_ids, block_table):
    """Scalar loops of mixed_attention (tiny inputs only)."""
    _, T, h_q, d = q.shape
    h_kv, page_size = k_pool.shape[1], k_pool.shape[2]
    G = h_q // h_kv
    qf, kf, vf = q.double().numpy(), k_pool.double().numpy(), v_pool.double().numpy()
    bt = block_table.numpy()
    out = np.zeros((T, h_q, d))
    scale = 1.0 / math.sqrt(d)
    cu = cu_seqlens.tolist()
    for b in range(slot_ids.shape[0]):
        c, s = int(kv_lens[b]), int(slot_ids[b])
        for i in range(cu[b + 1] - cu[b]):
            t = cu[b] + i
            for h in range(h_q):
                g = h // G
                keys = range(c + i + 1)
                sc = [sum(qf[0, t, h, x] * kf[bt[s, j // page_size], g, j % page_size, x]
                          for x in range(d)) * scale for j in keys]
                m = max(sc)
                w = [math.exp(v - m) for v in sc]
                tot = sum(w)
                for j, wj in zip(keys, w):
                    out[t, h] += (wj / tot) * vf[bt[s, j // page_size], g, j % page_size]
    return torch.from_numpy(out).float()


# ----------------------------------------------------------------------------- bytes

def decode_algorithmic_bytes(attended: list[int], h_q: int, h_kv: int, d: int,
                             page_size: int, elem: int = 2) -> int:
    """HBM bytes one decode call (append + load + merge) must move at minimum.

    K+V of every attended token, q in + o out, the int64 block-table entries
    walked, the appended K/V (read new rows + write pool rows), and the int64
    lens + slot ids.  Split partials are implementation overhead, not counted.
    """
    B = len(attended)
    kv = 2 * sum(attended) * h_kv * d * elem
    qo = 2 * B * h_q * d * elem
    bt = sum(-(-a // page_size) for a in attended) * 8
    append = 2 * B * h_kv * d * elem * 2
    idx = 16 * B
    return kv + qo + bt + append + idx
