"""Seeded random shapes through every kernel entry point, against the oracle.

Each case draws a batch (sizes, prior lengths, query rows), a head layout, a
head dim, a page size and a split count from a fixed seed, so the sweep is
reproducible and covers combinations the hand-picked tests do not: appends
must be bit-exact, attention within the tolerance of tests/conftest.py.
"""
import random

import pytest
import torch

from custom_inference_engine_amd import (append_tokens_qkv_rope, decode_qkv_rope_gqa_attention,
                                         mixed_gqa_attention)
from oracle import inputs
from oracle import paged_attention as ref
from tests.conftest import assert_attn_close
from tests.gpu_helpers import DEV, bits, gpu_decode_fused_step, gpu_decode_step, gpu_mixed_step, note
from tests.test_gpu_rope import _qkv, _tables

pytestmark = pytest.mark.gpu

HEADS = [(14, 2), (8, 2), (16, 1), (4, 4), (12, 4), (32, 8)]


def _decode_case(seed):
    rng = random.Random(seed)
    h_q, h_kv = rng.choice(HEADS)
    d = rng.choice([64, 128])
    ps = rng.choice([16, 16, 32, 64])
    hi = rng.choice([40, 600, 2500])
    B = rng.randint(1, 40 if hi <= 600 else 12)
    prior = [rng.randint(0, hi) for _ in range(B)]
    splits = rng.choice([None, 1, 2, 3, 7, 16])
    return inputs.make_case(prior, h_q=h_q, h_kv=h_kv, d=d, page_size=ps, seed=seed), splits


@pytest.mark.parametrize("seed", range(100, 124))
def test_random_decode_shapes(native_lib, seed):
    case, splits = _decode_case(seed)
    note(f"random decode seed={seed} B={case.B} heads={case.q.shape[2]}/{case.k_pool.shape[1]} "
         f"D={case.q.shape[3]} ps={case.page_size} splits={splits}")
    fused = seed % 2 == 0
    step = gpu_decode_fused_step if fused else gpu_decode_step
    kp, vp, o = step(case, n_splits=splits)
    ko, vo = case.appended_pools()
    assert torch.equal(bits(kp), bits(ko)) and torch.equal(bits(vp), bits(vo))
    want = ref.decode_attention(case.q, ko, vo, case.lens_pool[case.slot_ids] + 1, case.slot_ids,
                                case.block_table)
    assert_attn_close(o, want, what=f"random decode {seed}")


def _mixed_case(seed):
    rng = random.Random(seed)
    h_q, h_kv = rng.choice([h for h in HEADS if h[0] // h[1] <= 8])
    d = rng.choice([64, 128])
    ps = rng.choice([16, 32])
    B = rng.randint(1, 12)
    prior = [rng.choice([0, rng.randint(0, 1500)]) for _ in range(B)]
    new = [rng.choice([1, 1, rng.randint(1, 80), rng.randint(1, 300)]) for _ in range(B)]
    return inputs.make_case(prior, new, h_q=h_q, h_kv=h_kv, d=d, page_size=ps, seed=seed)


@pytest.mark.parametrize("seed", range(200, 216))
def test_random_mixed_shapes(native_lib, seed):
    case = _mixed_case(seed)
    note(f"random mixed seed={seed} B={case.B} rows={case.new_lens.tolist()} "
         f"heads={case.q.shape[2]}/{case.k_pool.shape[1]} D={case.q.shape[3]} ps={case.page_size}")
    kp, vp, o = gpu_mixed_step(case)
    ko, vo = case.appended_pools()
    assert torch.equal(bits(kp), bits(ko)) and torch.equal(bits(vp), bits(vo))
    want, written = ref.mixed_attention(case.q, ko, vo, case.cu_seqlens, case.kv_lens, case.slot_ids,
                                        case.block_table)
    assert_attn_close(o[written], want[written], what=f"random mixed {seed}")


@pytest.mark.parametrize("seed", range(300, 308))
def test_random_rope_paths(native_lib, seed):
    """Decode (one launch from the QKV rows) and token mode + mixed, against the oracle."""
    rng = random.Random(seed)
    h_q, h_kv = rng.choice([h for h in HEADS if h[0] // h[1] <= 8])
    d = rng.choice([64, 128])
    # decode
    B = rng.randint(1, 24)
    case = inputs.make_case([rng.randint(0, 900) for _ in range(B)], h_q=h_q, h_kv=h_kv, d=d, seed=seed)
    pos = case.lens_pool[case.slot_ids]
    cos, sin = _tables(pos, d)
    q_rot = ref.rope(case.q[0], cos, sin)[None]
    k_rot = ref.rope(case.k_new[0], cos, sin)[None]
    note(f"random rope decode seed={seed} B={B} heads={h_q}/{h_kv} D={d}")
    c = case.to(DEV)
    kp, vp = c.k_pool.clone(), c.v_pool.clone()
    o = decode_qkv_rope_gqa_attention(_qkv(case).to(DEV), cos[None].to(DEV), sin[None].to(DEV), kp, vp,
                                      c.lens_pool, c.slot_ids, c.block_table, num_heads=h_q)
    torch.cuda.synchronize()
    ko, vo = case.k_pool.clone(), case.v_pool.clone()
    ref.append_decode(ko, vo, k_rot, case.v_new, case.slot_ids, case.lens_pool, case.block_table)
    assert torch.equal(bits(kp), bits(ko)) and torch.equal(bits(vp), bits(vo))
    assert_attn_close(o[0], ref.decode_attention(q_rot, ko, vo, pos + 1, case.slot_ids, case.block_table),
                      what=f"random rope decode {seed}")
    # token mode + mixed
    n = rng.randint(1, 6)
    case = inputs.make_case([rng.randint(0, 700) for _ in range(n)], [rng.randint(1, 90) for _ in range(n)],
                            h_q=h_q, h_kv=h_kv, d=d, seed=seed + 1)
    T = case.q.shape[1]
    seq = torch.repeat_interleave(torch.arange(n), case.new_lens)
    pos = case.kv_lens[seq] + (torch.arange(T) - case.cu_seqlens[seq])
    cos, sin = _tables(pos, d)
    q_rot = ref.rope(case.q[0], cos, sin)[None]
    k_rot = ref.rope(case.k_new[0], cos, sin)[None]
    note(f"random rope tokens seed={seed} rows={case.new_lens.tolist()}")
    c = case.to(DEV)
    kp, vp = c.k_pool.clone(), c.v_pool.clone()
    q_out = append_tokens_qkv_rope(_qkv(case).to(DEV), cos[None].to(DEV), sin[None].to(DEV), kp, vp,
                                   c.pages, c.offsets, num_heads=h_q)
    o = mixed_gqa_attention(q_out, kp, vp, int(case.new_lens.max()), c.cu_seqlens, c.kv_lens, c.slot_ids,
                            c.block_table)
    torch.cuda.synchronize()
    ko, vo = case.k_pool.clone(), case.v_pool.clone()
    ref.append_tokens(ko, vo, k_rot, case.v_new, case.pages, case.offsets)
    assert torch.equal(bits(q_out), bits(q_rot))
    assert torch.equal(bits(kp), bits(ko)) and torch.equal(bits(vp), bits(vo))
    want, written = ref.mixed_attention(q_rot, ko, vo, case.cu_seqlens, case.kv_lens, case.slot_ids,
                                        case.block_table)
    assert_attn_close(o[0].float().cpu()[written], want[written], what=f"random rope mixed {seed}")
