"""QKV split + RoPE fused into the append kernels, against the oracle and the unfused path.

The fused decode launch (``cie_paged_decode_qkv_rope``) must give exactly what
the unfused fused-append decode gives on q / k rotated by the oracle (fp32,
rounded once): pools and o bit for bit, since the same attention code then
runs on identical operands.  The token-mode kernel
(``cie_kv_append_tokens_qkv_rope``) must write the oracle's rotated q and the
oracle's pools bit for bit.
"""
import pytest
import torch

from custom_inference_engine_amd import (append_tokens_qkv_rope, decode_append_gqa_attention,
                                         decode_qkv_rope_gqa_attention, mixed_gqa_attention)
from oracle import inputs
from oracle import paged_attention as ref
from tests.gpu_helpers import DEV, bits, note

pytestmark = pytest.mark.gpu


def _tables(positions: torch.Tensor, d: int, theta: float = 1e6):
    """Rotary tables as transformers' Qwen2RotaryEmbedding builds them (fp32, then fp16)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))
    ang = positions.float()[:, None] * inv_freq[None, :]
    emb = torch.cat([ang, ang], dim=-1)
    return emb.cos().half(), emb.sin().half()


def _qkv(case, pad: int = 0) -> torch.Tensor:
    """(1, T, (H_q + 2 H_kv) D) rows q | k | v; pad > 0 leaves a row stride wider than the width."""
    T, H_q, D = case.q.shape[1:]
    H_kv = case.k_pool.shape[1]
    width = (H_q + 2 * H_kv) * D
    buf = torch.zeros(1, T, width + pad, dtype=torch.float16)
    buf[0, :, :H_q * D] = case.q[0].reshape(T, -1)
    buf[0, :, H_q * D:(H_q + H_kv) * D] = case.k_new[0].reshape(T, -1)
    buf[0, :, (H_q + H_kv) * D:width] = case.v_new[0].reshape(T, -1)
    return buf[..., :width]


@pytest.mark.parametrize("h_q,h_kv,d,splits,pad", [
    (14, 2, 64, None, 0),
    (14, 2, 64, 3, 64),
    (14, 2, 64, 1, 0),
    (8, 2, 128, None, 0),
    (16, 1, 64, 5, 8),
])
def test_decode_qkv_rope_equals_rotated_unfused_path(native_lib, h_q, h_kv, d, splits, pad):
    case = inputs.make_case(None, h_q=h_q, h_kv=h_kv, d=d, random_lens=(0, 700, 11), seed=21)
    T = case.q.shape[1]
    pos = case.lens_pool[case.slot_ids]
    cos, sin = _tables(pos, d)
    q_rot = ref.rope(case.q[0], cos, sin)[None]
    k_rot = ref.rope(case.k_new[0], cos, sin)[None]
    note(f"decode qkv rope h_q={h_q} h_kv={h_kv} d={d} splits={splits} pad={pad}")
    c = case.to(DEV)
    kp1, vp1 = c.k_pool.clone(), c.v_pool.clone()
    o1 = decode_append_gqa_attention(q_rot.to(DEV), kp1, vp1, k_rot.to(DEV), c.v_new, c.lens_pool,
                                     c.slot_ids, c.block_table, num_programs=splits)
    kp2, vp2 = c.k_pool.clone(), c.v_pool.clone()
    o2 = decode_qkv_rope_gqa_attention(_qkv(case, pad).to(DEV), cos[None].to(DEV), sin[None].to(DEV),
                                       kp2, vp2, c.lens_pool, c.slot_ids, c.block_table,
                                       num_heads=h_q, num_programs=splits)
    torch.cuda.synchronize()
    assert o2.shape == (1, T, h_q, d)
    assert torch.equal(bits(kp2), bits(kp1)) and torch.equal(bits(vp2), bits(vp1))
    assert torch.equal(bits(o2), bits(o1))
    kp_ref, vp_ref = case.k_pool.clone(), case.v_pool.clone()
    ref.append_decode(kp_ref, vp_ref, k_rot, case.v_new, case.slot_ids, case.lens_pool, case.block_table)
    assert torch.equal(bits(kp2), bits(kp_ref)) and torch.equal(bits(vp2), bits(vp_ref))
    want = ref.decode_attention(q_rot, kp_ref, vp_ref, pos + 1, case.slot_ids, case.block_table)
    err = (o2[0].float().cpu() - want).abs()
    assert float(err.max()) <= 2e-3 + 1e-2 * float(want.abs().max())


def test_decode_qkv_rope_headline_shape(native_lib):
    """Config 2's shape (4097 attended: an odd tile per (sequence, kv head)) with positions 4096."""
    case = inputs.config2(seed=1)
    pos = case.lens_pool[case.slot_ids]
    cos, sin = _tables(pos, 64)
    q_rot = ref.rope(case.q[0], cos, sin)[None]
    k_rot = ref.rope(case.k_new[0], cos, sin)[None]
    note("decode qkv rope config 2")
    c = case.to(DEV)
    kp1, vp1 = c.k_pool.clone(), c.v_pool.clone()
    o1 = decode_append_gqa_attention(q_rot.to(DEV), kp1, vp1, k_rot.to(DEV), c.v_new, c.lens_pool,
                                     c.slot_ids, c.block_table)
    kp2, vp2 = c.k_pool.clone(), c.v_pool.clone()
    o2 = decode_qkv_rope_gqa_attention(_qkv(case).to(DEV), cos[None].to(DEV), sin[None].to(DEV), kp2, vp2,
                                       c.lens_pool, c.slot_ids, c.block_table, num_heads=14)
    torch.cuda.synchronize()
    assert torch.equal(bits(kp2), bits(kp1)) and torch.equal(bits(vp2), bits(vp1))
    assert torch.equal(bits(o2), bits(o1))


@pytest.mark.parametrize("prior,new,pad,h_q,h_kv,d", [
    ([0, 37, 300], [20, 1, 45], 0, 14, 2, 64),
    ([5, 0, 1000, 64, 3], [1, 64, 17, 1, 33], 16, 14, 2, 64),
    ([3, 130], [40, 2], 0, 8, 2, 128),
    ([0, 17], [19, 5], 8, 4, 4, 64),
])
def test_append_tokens_qkv_rope_matches_oracle(native_lib, prior, new, pad, h_q, h_kv, d):
    case = inputs.make_case(prior, new, h_q=h_q, h_kv=h_kv, d=d, seed=9)
    T, H_q, D = case.q.shape[1:]
    seq = torch.repeat_interleave(torch.arange(len(prior)), case.new_lens)
    pos = case.kv_lens[seq] + (torch.arange(T) - case.cu_seqlens[seq])
    cos, sin = _tables(pos, D)
    q_rot = ref.rope(case.q[0], cos, sin)[None]
    k_rot = ref.rope(case.k_new[0], cos, sin)[None]
    note(f"token rope append prior={prior} new={new}")
    c = case.to(DEV)
    kp, vp = c.k_pool.clone(), c.v_pool.clone()
    q_out = append_tokens_qkv_rope(_qkv(case, pad).to(DEV), cos[None].to(DEV), sin[None].to(DEV), kp, vp,
                                   c.pages, c.offsets, num_heads=H_q)
    torch.cuda.synchronize()
    assert torch.equal(bits(q_out), bits(q_rot))
    kp_ref, vp_ref = case.k_pool.clone(), case.v_pool.clone()
    ref.append_tokens(kp_ref, vp_ref, k_rot, case.v_new, case.pages, case.offsets)
    assert torch.equal(bits(kp), bits(kp_ref)) and torch.equal(bits(vp), bits(vp_ref))
    # the mixed kernel on the kernel's q equals it on the oracle's q
    max_seqlen = int(case.new_lens.max())
    o1 = mixed_gqa_attention(q_out, kp, vp, max_seqlen, c.cu_seqlens, c.kv_lens, c.slot_ids, c.block_table)
    o2 = mixed_gqa_attention(q_rot.to(DEV), kp, vp, max_seqlen, c.cu_seqlens, c.kv_lens, c.slot_ids,
                             c.block_table)
    torch.cuda.synchronize()
    assert torch.equal(bits(o1), bits(o2))


def test_rope_entry_points_reject_bad_layouts(native_lib):
    case = inputs.make_case([10], seed=2)
    c = case.to(DEV)
    cos, sin = _tables(torch.tensor([10]), 64)
    qkv = _qkv(case).to(DEV)
    with pytest.raises(AssertionError):  # wrong width for the head counts
        decode_qkv_rope_gqa_attention(qkv[..., :-64], cos[None].to(DEV), sin[None].to(DEV), c.k_pool,
                                      c.v_pool, c.lens_pool, c.slot_ids, c.block_table, num_heads=14)
    with pytest.raises(AssertionError):  # one cos row per token
        append_tokens_qkv_rope(qkv, torch.cat([cos, cos])[None].to(DEV), sin[None].to(DEV), c.k_pool,
                               c.v_pool, c.pages, c.offsets, num_heads=14)
