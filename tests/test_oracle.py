"""Pins for the CPU oracle (no GPU).

Every oracle function is checked against something that is not a retyping of
its own formula: scalar brute-force loops, torch's scaled_dot_product_attention
(a library routine) on contiguous K/V, closed forms, invariants, and the
golden fixtures.  Planted mistakes (mutants of the oracle, built here on the
CPU) must fail the same checks, which shows the checks can see the mistakes
that matter: a wrong scale, head mapping, causal offset, length or page walk.
"""
import json
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import inputs, paged_attention as ref

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
TIGHT = 1e-5


def _decode(case, fn=ref.decode_attention):
    kp, vp = case.appended_pools()
    return fn(case.q, kp, vp, case.attended, case.slot_ids, case.block_table)


def _mixed(case, fn=ref.mixed_attention):
    kp, vp = case.appended_pools()
    return fn(case.q, kp, vp, case.cu_seqlens, case.kv_lens, case.slot_ids, case.block_table)


# ----------------------------------------------------------------------------- mutants

def _mut_decode_head_mod(q, k_pool, v_pool, lens, slot_ids, block_table):
    """Planted mistake: query head h reads kv head h % H_kv instead of h // G."""
    h_q, h_kv = q.shape[2], k_pool.shape[1]
    perm = [h % h_kv * (h_q // h_kv) + h // h_kv for h in range(h_q)]
    inv = [perm.index(i) for i in range(h_q)]
    out = ref.decode_attention(q[:, :, inv], k_pool, v_pool, lens, slot_ids, block_table)
    return out[:, perm]


def _mut_decode_scale(q, k_pool, v_pool, lens, slot_ids, block_table):
    """Planted mistake: scores multiplied by sqrt(D) instead of 1/sqrt(D)."""
    d = q.shape[-1]
    return ref.decode_attention((q.float() * d).half(), k_pool, v_pool, lens, slot_ids, block_table)


def _mut_decode_short(q, k_pool, v_pool, lens, slot_ids, block_table):
    """Planted mistake: the appended token is not attended (lens - 1)."""
    return ref.decode_attention(q, k_pool, v_pool, (lens - 1).clamp(min=0), slot_ids, block_table)


def _mut_decode_identity_pages(q, k_pool, v_pool, lens, slot_ids, block_table):
    """Planted mistake: logical page used as physical page (block table ignored)."""
    bt = torch.arange(block_table.shape[1]).expand_as(block_table).contiguous()
    bt = bt.clamp(max=k_pool.shape[0] - 1)
    return ref.decode_attention(q, k_pool, v_pool, lens, slot_ids, bt)


def _mut_mixed_strict(q, k_pool, v_pool, cu, kv_lens, slot_ids, bt):
    """Planted mistake: causal rule j < kv_len + i (the diagonal dropped) — emulated by a
    one-step-earlier prior length for all rows but the first key."""
    out, written = ref.mixed_attention(q, k_pool, v_pool, cu, (kv_lens - 1).clamp(min=0), slot_ids, bt)
    return out, written


def _mut_mixed_no_prior(q, k_pool, v_pool, cu, kv_lens, slot_ids, bt):
    """Planted mistake: the prior KV length is ignored (causal from position 0)."""
    return ref.mixed_attention(q, k_pool, v_pool, cu, torch.zeros_like(kv_lens), slot_ids, bt)


DECODE_MUTANTS = [_mut_decode_head_mod, _mut_decode_scale, _mut_decode_short,
                  _mut_decode_identity_pages]
MIXED_MUTANTS = [_mut_mixed_strict, _mut_mixed_no_prior]


# ----------------------------------------------------------------------------- append

@pytest.mark.parametrize("seed", [0, 1])
def test_append_decode_matches_scalar_loop(seed):
    case = inputs.make_case([0, 15, 16, 31, 47], seed=seed)
    kp, vp = case.k_pool.clone(), case.v_pool.clone()
    ref.append_decode(kp, vp, case.k_new, case.v_new, case.slot_ids, case.lens_pool, case.block_table)
    kb, vb = case.k_pool.clone(), case.v_pool.clone()
    ref.append_decode_bruteforce(kb, vb, case.k_new, case.v_new, case.slot_ids, case.lens_pool,
                                 case.block_table)
    assert torch.equal(kp.view(torch.int16), kb.view(torch.int16))
    assert torch.equal(vp.view(torch.int16), vb.view(torch.int16))
    # the token-mode restatement with the mixed_module.py page / offset recipe agrees
    kt, vt = case.appended_pools()
    assert torch.equal(kp.view(torch.int16), kt.view(torch.int16))
    assert torch.equal(vp.view(torch.int16), vt.view(torch.int16))
    # exactly one row per sequence changed, at (block_table[s, pos // 16], pos % 16)
    changed = (kp != case.k_pool).any(dim=-1).any(dim=1).nonzero().tolist()
    want = sorted([int(case.block_table[s, int(case.lens_pool[s]) // 16]), int(case.lens_pool[s]) % 16]
                  for s in case.slot_ids.tolist())
    assert sorted(changed) == want


def test_append_padding_rows_land_on_page0():
    """Padding slot 0 (lens 0, block-table row 0) writes page 0 offset 0 (storage.py:20, metadata.py:33-37)."""
    case = inputs.make_case([20, 40], seed=2)
    slot_ids = torch.tensor([1, 0, 2, 0])
    k_new = torch.randn(1, 4, 2, 64).half()
    kp, vp = case.k_pool.clone(), case.v_pool.clone()
    ref.append_decode(kp, vp, k_new, k_new, slot_ids, case.lens_pool, case.block_table)
    changed_pages = set((kp != case.k_pool).any(dim=-1).any(dim=-1).any(dim=-1).nonzero().flatten().tolist())
    real = {int(case.block_table[s, int(case.lens_pool[s]) // 16]) for s in (1, 2)}
    assert changed_pages == real | {0}


def test_mixed_pages_offsets_recipe():
    case = inputs.make_case([3, 0, 30], [5, 2, 4], seed=4)
    pages, offsets, pos = ref.mixed_pages_offsets(case.lens_pool, case.block_table, case.slot_ids,
                                                  case.cu_seqlens, 16)
    t = 0
    for b, s in enumerate(case.slot_ids.tolist()):
        for i in range(int(case.new_lens[b])):
            p = int(case.kv_lens[b]) + i
            assert int(pos[t]) == p
            assert int(pages[t]) == int(case.block_table[s, p // 16])
            assert int(offsets[t]) == p % 16
            t += 1
    assert t == case.T


# ----------------------------------------------------------------------------- decode

@pytest.mark.parametrize("seed", [0, 1, 2])
def test_decode_matches_bruteforce(seed):
    case = inputs.make_case(None, random_lens=(0, 40, 3), seed=seed)
    kp, vp = case.appended_pools()
    args = (case.q, kp, vp, case.attended, case.slot_ids, case.block_table)
    brute = ref.decode_attention_bruteforce(*args)
    assert (ref.decode_attention(*args) - brute).abs().max() < TIGHT
    for mutant in DECODE_MUTANTS:
        assert (mutant(*args) - brute).abs().max() > 1e-2, mutant.__name__


def test_decode_matches_sdpa_on_contiguous_kv():
    """Library routine: SDPA (GQA via enable_gqa) on K/V laid out contiguously."""
    case = inputs.make_case([63], seed=7, h_q=8, h_kv=2, d=64)
    kp, vp = case.appended_pools()
    L = int(case.attended[0])
    n = -(-L // 16)
    pages = case.block_table[1, :n]
    K = kp[pages].float().permute(1, 0, 2, 3).reshape(2, -1, 64)[:, :L]
    V = vp[pages].float().permute(1, 0, 2, 3).reshape(2, -1, 64)[:, :L]
    want = F.scaled_dot_product_attention(case.q[0].float().permute(1, 0, 2)[None], K[None], V[None],
                                          enable_gqa=True)[0, :, 0]
    got = _decode(case)[0]
    assert (got - want).abs().max() < TIGHT


def test_decode_closed_forms():
    case = inputs.make_case([0, 9], seed=8)
    kp, vp = case.appended_pools()
    # single key: softmax is 1, o = v0 exactly (fp16 value, fp32 math)
    out = ref.decode_attention(case.q, kp, vp, case.attended, case.slot_ids, case.block_table)
    v0 = vp[case.block_table[1, 0], :, 0].float()
    assert torch.allclose(out[0], v0.repeat_interleave(7, dim=0), atol=1e-6)
    # empty sequence: o = 0 (the -inf guard, kernels/decode_attention.py:260-264)
    out0 = ref.decode_attention(case.q, kp, vp, torch.tensor([0, 10]), case.slot_ids, case.block_table)
    assert torch.count_nonzero(out0[0]) == 0
    # identical keys: uniform weights, o = mean of V over the 10 tokens
    kp2 = kp.clone()
    pages = case.block_table[2, :1]
    kp2[pages] = kp2[pages][:, :, :1].expand(-1, -1, 16, -1)
    out2 = ref.decode_attention(case.q, kp2, vp, case.attended, case.slot_ids, case.block_table)
    Vs = vp[pages].float()[0, :, :10]  # (H_kv, 10, D)
    assert torch.allclose(out2[1], Vs.mean(dim=1).repeat_interleave(7, dim=0), atol=1e-5)


def test_decode_page_permutation_invariance():
    case = inputs.make_case([37, 70], seed=9)
    kp, vp = case.appended_pools()
    base = ref.decode_attention(case.q, kp, vp, case.attended, case.slot_ids, case.block_table)
    g = torch.Generator().manual_seed(1)
    n = kp.shape[0]
    perm = torch.cat([torch.zeros(1, dtype=torch.long), torch.randperm(n - 1, generator=g) + 1])
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(n)
    kp2, vp2 = torch.empty_like(kp), torch.empty_like(vp)
    kp2[inv], vp2[inv] = kp, vp  # physical page p moves to inv[p]
    bt2 = inv[case.block_table]
    moved = ref.decode_attention(case.q, kp2, vp2, case.attended, case.slot_ids, bt2)
    assert torch.equal(base, moved)


@pytest.mark.parametrize("P", [1, 3, 4, 16, 40])
def test_reference_splitkv_algorithm_equals_exact_softmax(P):
    """The reference's interleaved split + LSE merge (fp16 P) lands within the parity bar."""
    case = inputs.make_case([0, 5, 100, 300], seed=11)
    kp, vp = case.appended_pools()
    args = (case.q, kp, vp, case.attended, case.slot_ids, case.block_table)
    exact = ref.decode_attention(*args)
    split = ref.decode_attention_splitkv(*args, num_programs=P)
    err = (split - exact).abs()
    assert float(err.max()) < 2e-3
    # splits with no rows (P*16 > L) leave m = -inf and do not disturb the merge
    assert torch.isfinite(split).all()


def test_reference_splitkv_empty_sequence_is_zero():
    case = inputs.make_case([10], seed=12)
    kp, vp = case.appended_pools()
    out = ref.decode_attention_splitkv(case.q, kp, vp, torch.tensor([0]), case.slot_ids,
                                       case.block_table, num_programs=4)
    assert torch.count_nonzero(out) == 0


# ----------------------------------------------------------------------------- mixed

@pytest.mark.parametrize("seed", [0, 1])
def test_mixed_matches_bruteforce(seed):
    case = inputs.make_case([0, 7, 33], [9, 1, 4], seed=seed)
    out, written = _mixed(case)
    kp, vp = case.appended_pools()
    args = (case.q, kp, vp, case.cu_seqlens, case.kv_lens, case.slot_ids, case.block_table)
    brute = ref.mixed_attention_bruteforce(*args)
    assert written.all()
    assert (out - brute).abs().max() < TIGHT
    for mutant in MIXED_MUTANTS:
        mo, _ = mutant(*args)
        assert (mo - brute).abs().max() > 1e-2, mutant.__name__


def test_mixed_prefill_from_empty_is_textbook_causal():
    """kv_len = 0: plain causal self-attention (SDPA is_causal on contiguous K/V)."""
    case = inputs.make_case([0], [40], seed=13, h_q=4, h_kv=4)
    out, _ = _mixed(case)
    kp, vp = case.appended_pools()
    pages = case.block_table[1, :3]
    K = kp[pages].float().permute(1, 0, 2, 3).reshape(4, -1, 64)[:, :40]
    V = vp[pages].float().permute(1, 0, 2, 3).reshape(4, -1, 64)[:, :40]
    Q = case.q[0].float().permute(1, 0, 2)
    want = F.scaled_dot_product_attention(Q[None], K[None], V[None], is_causal=True)[0].permute(1, 0, 2)
    assert (out - want).abs().max() < TIGHT


def test_mixed_single_row_equals_decode():
    case = inputs.make_case([0, 16, 200], seed=14)
    out, _ = _mixed(case)
    dec = _decode(case)
    assert (out - dec).abs().max() < TIGHT


def test_mixed_skips_empty_sequences():
    case = inputs.make_case([5, 9, 0], [3, 0, 2], seed=15)
    out, written = _mixed(case)
    assert written.all() and written.numel() == 5
    # the empty middle sequence contributes no rows and does not shift the others
    assert case.cu_seqlens.tolist() == [0, 3, 3, 5]
    dec = _decode(inputs.make_case([9], seed=15))
    assert dec.shape[0] == 1


def test_mixed_chunked_prefill_equals_one_shot():
    """A prefill split into chunks (kv_len resumes) equals one causal pass."""
    one = inputs.make_case([0], [48], seed=16)
    out1, _ = _mixed(one)
    kp, vp = one.appended_pools()
    for c0, c1 in [(0, 16), (16, 37), (37, 48)]:
        cu = torch.tensor([0, c1 - c0])
        o, _ = ref.mixed_attention(one.q[:, c0:c1], kp, vp, cu, torch.tensor([c0]), one.slot_ids,
                                   one.block_table)
        assert (o - out1[c0:c1]).abs().max() < TIGHT


# ----------------------------------------------------------------------------- golden

def _load_golden(name):
    z = np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False)
    return json.loads(str(z["meta"])), z


@pytest.mark.parametrize("name", ["config1_decode", "decode_edges", "mixed_small"])
def test_golden_fixture_reproduces(name):
    from tests.golden.make_golden import INPUT_FIELDS, build_case, digest

    meta, z = _load_golden(name)
    case = build_case(meta["spec"])
    for f in INPUT_FIELDS:
        assert digest(getattr(case, f)) == meta["digests"][f], f"input recipe drifted: {f}"
    kp, vp = case.appended_pools()
    assert digest(kp) == meta["pool_digest_k"] and digest(vp) == meta["pool_digest_v"]
    if meta["kind"] == "decode":
        out = _decode(case)
    else:
        out, written = _mixed(case)
        assert np.array_equal(written.numpy(), z["written"])
    assert np.abs(out.numpy() - z["out"]).max() < TIGHT


def test_algorithmic_bytes_headline():
    """67,339,008 B for B=32, attend 4097, 14/2 heads, D=64 (the published target's formula)."""
    assert ref.decode_algorithmic_bytes([4097] * 32, 14, 2, 64, 16) == 67_339_008
    assert ref.decode_algorithmic_bytes([16385] * 16, 14, 2, 64, 16) == 134_431_104
    assert ref.decode_algorithmic_bytes([129], 14, 2, 64, 16) == 70_744


# ----------------------------------------------------------------------------- rope

def _rope_inputs(seed, T=5, H=3, D=64):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(T, H, D, generator=g) * 2).half()
    ang = torch.rand(T, D // 2, generator=g, dtype=torch.float64) * 50
    ang = torch.cat([ang, ang], dim=-1)
    return x, ang.cos().half(), ang.sin().half()


@pytest.mark.parametrize("seed", [0, 1])
def test_rope_matches_transformers_apply_rotary_pos_emb(seed):
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb
    x, cos, sin = _rope_inputs(seed)
    # transformers layout: (batch, heads, T, D) with cos / sin (batch, T, D)
    q = x.float().permute(1, 0, 2)[None]
    qe, _ = apply_rotary_pos_emb(q, q, cos.float()[None], sin.float()[None], unsqueeze_dim=1)
    want = qe[0].permute(1, 0, 2).half()
    assert torch.equal(ref.rope(x, cos, sin), want)


def test_rope_matches_the_compiled_reference_step():
    """What the reference's compiled step stores: transformers' apply_rotary_pos_emb
    on fp16 q / k / cos / sin, compiled by torch.compile's inductor (here its CPU
    code generation, which like its GPU code generation computes an fp16 pointwise
    chain in fp32 and rounds once at the store), equals the oracle's rope bit for
    bit — and differs from the same function run eagerly in fp16, which rounds
    after every operation."""
    import torch._dynamo
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb

    x, cos, sin = _rope_inputs(4, T=16, H=4)
    q = x.permute(1, 0, 2)[None].contiguous()  # (batch, heads, T, D), fp16
    c, s = cos[None], sin[None]

    def step(q, k, c, s):
        return apply_rotary_pos_emb(q, k, c, s, unsqueeze_dim=1)

    torch._dynamo.reset()
    qc, kc = torch.compile(step, backend="inductor", fullgraph=True)(q, q, c, s)
    torch._dynamo.reset()
    want = ref.rope(x, cos, sin)
    assert torch.equal(qc[0].permute(1, 0, 2), want)
    assert torch.equal(kc[0].permute(1, 0, 2), want)
    qe, _ = step(q, q, c, s)  # eager fp16
    assert not torch.equal(qe[0].permute(1, 0, 2), want)


def test_rope_identity_at_angle_zero_and_rotation_closed_form():
    x, _, _ = _rope_inputs(2)
    T, H, D = x.shape
    one, zero = torch.ones(T, D).half(), torch.zeros(T, D).half()
    assert torch.equal(ref.rope(x, one, zero), x)
    # a quarter turn maps (a, b) -> (-b, a) exactly
    y = ref.rope(x, zero, one)
    half = D // 2
    assert torch.equal(y[..., :half], -x[..., half:])
    assert torch.equal(y[..., half:], x[..., :half])


def test_rope_pin_catches_a_flipped_rotate_half():
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb
    x, cos, sin = _rope_inputs(3)
    xf = x.float()
    half = xf.shape[-1] // 2
    wrong = (xf * cos.float()[:, None] + torch.cat([xf[..., half:], -xf[..., :half]], -1)
             * sin.float()[:, None]).half()
    q = x.float().permute(1, 0, 2)[None]
    qe, _ = apply_rotary_pos_emb(q, q, cos.float()[None], sin.float()[None], unsqueeze_dim=1)
    assert not torch.equal(wrong, qe[0].permute(1, 0, 2).half())
