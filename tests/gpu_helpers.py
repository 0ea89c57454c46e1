"""Shared plumbing for the GPU parity tests: run the HIP path on an oracle case."""
import sys

import torch

from custom_inference_engine_amd import (decode_append_gqa_attention, decode_gqa_attention, kv_append_decode,
                                         kv_append_tokens, mixed_gqa_attention)
from oracle import paged_attention as ref

DEV = "cuda"


def note(msg: str) -> None:
    """Name the case before each GPU step (a fault ends the process)."""
    print(f"[gpu] {msg}", file=sys.stderr, flush=True)


def bits(t: torch.Tensor) -> torch.Tensor:
    return t.detach().cpu().contiguous().view(torch.int16)


def err_word() -> torch.Tensor:
    return torch.zeros(1, dtype=torch.int32, device=DEV)


def gpu_decode_step(case, n_splits=None, err=None):
    """Decode append + split-KV attention on the GPU; returns (k_pool, v_pool, o) on the CPU."""
    c = case.to(DEV)
    kp, vp = c.k_pool.clone(), c.v_pool.clone()
    kv_append_decode(kp, vp, c.k_new, c.v_new, c.slot_ids, c.lens_pool, c.block_table, err=err)
    o = decode_gqa_attention(c.q, kp, vp, c.attended, c.slot_ids, c.block_table,
                             num_programs=n_splits, err=err)
    torch.cuda.synchronize()
    return kp.cpu(), vp.cpu(), o[0].float().cpu()


def gpu_decode_fused_step(case, n_splits=None, err=None):
    """KV append fused into the decode launch; returns (k_pool, v_pool, o) on the CPU."""
    c = case.to(DEV)
    kp, vp = c.k_pool.clone(), c.v_pool.clone()
    o = decode_append_gqa_attention(c.q, kp, vp, c.k_new, c.v_new, c.lens_pool, c.slot_ids,
                                    c.block_table, num_programs=n_splits, err=err)
    torch.cuda.synchronize()
    return kp.cpu(), vp.cpu(), o[0].float().cpu()


def gpu_mixed_step(case, max_seqlen=None, err=None):
    """Token-mode append + varlen mixed attention on the GPU; returns (k_pool, v_pool, o)."""
    c = case.to(DEV)
    kp, vp = c.k_pool.clone(), c.v_pool.clone()
    kv_append_tokens(kp, vp, c.k_new, c.v_new, c.pages, c.offsets, err=err)
    if max_seqlen is None:
        max_seqlen = int(case.new_lens.max()) if case.B else 0
    o = mixed_gqa_attention(c.q, kp, vp, max_seqlen, c.cu_seqlens, c.kv_lens, c.slot_ids,
                            c.block_table, err=err)
    torch.cuda.synchronize()
    return kp.cpu(), vp.cpu(), o[0].float().cpu()


def oracle_decode(case):
    kp, vp = case.appended_pools()
    return ref.decode_attention(case.q, kp, vp, case.attended, case.slot_ids, case.block_table)


def oracle_mixed(case):
    kp, vp = case.appended_pools()
    return ref.mixed_attention(case.q, kp, vp, case.cu_seqlens, case.kv_lens, case.slot_ids,
                               case.block_table)
