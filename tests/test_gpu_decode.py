"""Split-KV paged decode on the GPU against the fp32 oracle (tolerance 2e-3 abs / 1e-2 rel)."""
import json
import os

import numpy as np
import pytest
import torch

from custom_inference_engine_amd import decode_gqa_attention
from oracle import inputs
from tests.conftest import assert_attn_close
from tests.golden.make_golden import INPUT_FIELDS, build_case, digest
from tests.gpu_helpers import DEV, bits, err_word, gpu_decode_fused_step, gpu_decode_step, note, oracle_decode

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.mark.parametrize("name", ["config1_decode", "decode_edges"])
def test_decode_matches_golden_fixture(native_lib, name):
    z = np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False)
    meta = json.loads(str(z["meta"]))
    case = build_case(meta["spec"])
    for f in INPUT_FIELDS:
        assert digest(getattr(case, f)) == meta["digests"][f], f
    note(f"golden {name}")
    kp, vp, o = gpu_decode_step(case, n_splits=case.meta.get("n_splits"))
    assert digest(kp) == meta["pool_digest_k"] and digest(vp) == meta["pool_digest_v"]
    assert_attn_close(o, torch.from_numpy(z["out"]), what=name)


@pytest.mark.parametrize("make,splits", [
    (lambda: inputs.config1(), 4),
    (lambda: inputs.config2(seed=0), None),
    (lambda: inputs.config2(seed=0), 16),
    (lambda: inputs.config2(seed=1, fixed=False), None),
    (lambda: inputs.config2(seed=2, fixed=False), 16),
    (lambda: inputs.config4(), 16),
], ids=["cfg1-p4", "cfg2-auto", "cfg2-p16", "cfg2var-auto", "cfg2var-p16", "cfg4-p16"])
def test_decode_baseline_configs(native_lib, make, splits):
    case = make()
    note(f"decode B={case.B} max_len={int(case.attended.max())} splits={splits}")
    kp, vp, o = gpu_decode_step(case, n_splits=splits)
    ko, vo = case.appended_pools()
    assert torch.equal(bits(kp), bits(ko)) and torch.equal(bits(vp), bits(vo))
    assert_attn_close(o, oracle_decode(case), what="decode")


@pytest.mark.parametrize("splits", [1, 2, 3, 7, 16, 64])
def test_decode_split_count_does_not_change_result(native_lib, splits):
    case = inputs.make_case([0, 1, 17, 250, 1000], seed=21)
    note(f"decode split sweep {splits}")
    _, _, o = gpu_decode_step(case, n_splits=splits)
    assert_attn_close(o, oracle_decode(case), what=f"splits={splits}")


def test_decode_edge_lengths(native_lib):
    """Attended lengths at and around tile / pair / page boundaries, and zero."""
    prior = [0, 1, 14, 15, 16, 30, 31, 32, 33, 47, 63, 64, 65, 127, 128]
    case = inputs.make_case(prior, seed=22)
    note("decode edges")
    _, _, o = gpu_decode_step(case, n_splits=3)
    assert_attn_close(o, oracle_decode(case), what="edges")
    # an empty sequence gives exactly 0 (kernels/decode_attention.py:260-264)
    c = case.to(DEV)
    lens = c.attended.clone()
    lens[2] = 0
    out = decode_gqa_attention(c.q, c.k_pool, c.v_pool, lens, c.slot_ids, c.block_table, num_programs=5)
    assert torch.count_nonzero(out[0, 2]) == 0
    # one token: o = v of that token (up to fp16 rounding of the output)
    lens[3] = 1
    out = decode_gqa_attention(c.q, c.k_pool, c.v_pool, lens, c.slot_ids, c.block_table, num_programs=5)
    v0 = case.v_pool[case.block_table[4, 0], :, 0].float().repeat_interleave(7, dim=0)
    assert torch.equal(out[0, 3].float().cpu(), v0.half().float())


@pytest.mark.parametrize("h_q,h_kv,d,ps", [
    (8, 8, 64, 16), (16, 1, 64, 16), (28, 4, 64, 16), (14, 2, 128, 16), (14, 2, 64, 64), (7, 1, 64, 32),
])
def test_decode_head_geometries(native_lib, h_q, h_kv, d, ps):
    case = inputs.make_case([5, 100, 333], seed=23, h_q=h_q, h_kv=h_kv, d=d, page_size=ps)
    note(f"decode geometry {h_q}/{h_kv} D={d} ps={ps}")
    kp, vp, o = gpu_decode_step(case, n_splits=4)
    ko, vo = case.appended_pools()
    assert torch.equal(bits(kp), bits(ko))
    assert_attn_close(o, oracle_decode(case), what="geometry")


def test_decode_is_deterministic(native_lib):
    case = inputs.make_case([700, 64, 3000], seed=24)
    note("decode determinism")
    o1 = gpu_decode_step(case)[2]
    o2 = gpu_decode_step(case)[2]
    assert torch.equal(o1, o2)


def test_decode_length_overflow_is_clamped_and_flagged(native_lib):
    case = inputs.make_case([40], seed=25, bt_width=None)
    note("decode overflow flag")
    c = case.to(DEV)
    err = err_word()
    cap = c.block_table.shape[1] * 16
    lens = torch.tensor([cap + 100], device=DEV)
    decode_gqa_attention(c.q, c.k_pool, c.v_pool, lens, c.slot_ids, c.block_table, num_programs=2, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) & 2


def test_decode_rejects_cpu_tensors():
    """No CPU fallback: the product path raises on host tensors."""
    case = inputs.make_case([10], seed=26)
    with pytest.raises(RuntimeError, match="HIP device"):
        decode_gqa_attention(case.q, case.k_pool, case.v_pool, case.attended, case.slot_ids,
                             case.block_table, num_programs=2)


# ----------------------------------------------------------------------------- fused append + decode

@pytest.mark.parametrize("make,splits", [
    (lambda: inputs.config1(), 4),
    (lambda: inputs.config2(seed=0), None),
    (lambda: inputs.config2(seed=3, fixed=False), 16),
    (lambda: inputs.config4(), 16),
    (lambda: inputs.make_case([0, 1, 14, 15, 16, 30, 31, 32, 47, 63, 64, 127], seed=27), 3),
    (lambda: inputs.make_case([0, 1, 14, 15, 16, 30, 31, 32, 47, 63, 64, 127], seed=27), 1),
    (lambda: inputs.make_case([5, 100, 333], seed=28, h_q=16, h_kv=1, d=128, page_size=32), 5),
], ids=["cfg1", "cfg2", "cfg2var", "cfg4", "edges-p3", "edges-p1", "g16-d128-ps32"])
def test_fused_append_decode(native_lib, make, splits):
    case = make()
    note(f"fused decode B={case.B} splits={splits}")
    err = err_word()
    kp, vp, o = gpu_decode_fused_step(case, n_splits=splits, err=err)
    ko, vo = case.appended_pools()
    assert torch.equal(bits(kp), bits(ko)) and torch.equal(bits(vp), bits(vo)), "append not bit-exact"
    assert_attn_close(o, oracle_decode(case), what="fused decode")
    assert int(err.item()) == 0


def test_fused_matches_two_launch_path_bitwise(native_lib):
    """One launch (append fused) == decode_update + decode op, bit for bit."""
    case = inputs.make_case([7, 90, 1000, 4095], seed=29)
    note("fused vs two-launch")
    kf, vf, of = gpu_decode_fused_step(case, n_splits=4)
    k2, v2, o2 = gpu_decode_step(case, n_splits=4)
    assert torch.equal(bits(kf), bits(k2)) and torch.equal(bits(vf), bits(v2))
    assert torch.equal(of, o2)


def test_decode_counters_return_to_zero(native_lib):
    """Every call leaves the arrival counters zero, so the buffer is reused without clearing."""
    case = inputs.make_case([300, 1, 2000], seed=30)
    note("split counters")
    c = case.to(DEV)
    kp, vp = (t.to(DEV) for t in case.appended_pools())
    ctr = torch.zeros(2 * case.B * 2, dtype=torch.int32, device=DEV)  # arrival + stale words
    outs = []
    for splits in (7, 7, 3, 16):
        o = decode_gqa_attention(c.q, kp, vp, c.attended, c.slot_ids, c.block_table,
                                 num_programs=splits, counters=ctr)
        outs.append(o.clone())
        torch.cuda.synchronize()
        assert torch.count_nonzero(ctr) == 0
    assert torch.equal(outs[0], outs[1])
    for o in outs:
        assert_attn_close(o[0].float().cpu(), oracle_decode(case), what="counters")


def test_decode_stale_counter_is_flagged_and_cleared(native_lib):
    """An arrival word left at n_splits or more (a caller's unzeroed buffer) raises
    CIE_ERRBIT_SPLIT; every split of that (sequence, kv head) sees it stale, so the
    call puts the word back to zero and the next call is correct again.  The other
    (sequence, kv head) groups of the stale call are unaffected."""
    case = inputs.make_case([300, 1, 2000], seed=31)
    note("decode stale counter")
    c = case.to(DEV)
    kp, vp = (t.to(DEV) for t in case.appended_pools())
    want = oracle_decode(case)
    S, n = 4, case.B * 2
    ctr = torch.zeros(2 * n, dtype=torch.int32, device=DEV)
    ctr[2 * 1 + 1] = S + 5  # arrival word of (sequence 1, kv head 1)
    err = err_word()
    o = decode_gqa_attention(c.q, kp, vp, c.attended, c.slot_ids, c.block_table, num_programs=S,
                             counters=ctr, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 8, "CIE_ERRBIT_SPLIT expected"
    assert torch.count_nonzero(ctr) == 0, ctr.tolist()
    fine = [(b, h) for b in range(case.B) for h in range(14) if not (b == 1 and h >= 7)]
    got = o[0].float().cpu()
    for b, h in fine:
        assert_attn_close(got[b, h], want[b, h], what=f"untouched group b={b} h={h}")
    err.zero_()
    o = decode_gqa_attention(c.q, kp, vp, c.attended, c.slot_ids, c.block_table, num_programs=S,
                             counters=ctr, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    assert torch.count_nonzero(ctr) == 0
    assert_attn_close(o[0].float().cpu(), want, what="call after the stale one")


def test_decode_ignores_block_table_entries_past_the_sequence(native_lib):
    """The kernel fetches page ids ahead of knowing each sequence's length; entries of
    a block-table row past the sequence's pages may hold anything (here: -7 and ids
    beyond the pool) and must neither raise CIE_ERRBIT_PAGE nor change the result."""
    case = inputs.make_case([30, 300, 1000, 5], seed=54)
    note("decode garbage past the sequence")
    bt = case.block_table.clone()
    for b in range(case.B):
        s = int(case.slot_ids[b])
        used = -(-int(case.attended[b]) // 16)
        bt[s, used:] = torch.where(torch.arange(bt.shape[1] - used) % 2 == 0, -7, bt.shape[1] + 100)
    c = case.to(DEV)
    kp, vp = (t.to(DEV) for t in case.appended_pools())
    err = err_word()
    o = decode_gqa_attention(c.q, kp, vp, c.attended, c.slot_ids, bt.to(DEV), num_programs=4, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    assert_attn_close(o[0].float().cpu(), oracle_decode(case), what="garbage past the sequence")


def test_decode_counter_preloaded_negative_is_flagged_then_reset(native_lib):
    """A word just below zero (-1) is flagged on the call that finds it; since the
    stale value then lands inside [0, n_splits) the caller re-zeroes the counters
    (reset_split_counters for the library's own buffer), and the next call is
    correct with no error bit."""
    from custom_inference_engine_amd.attn.core import reset_split_counters, split_counters

    case = inputs.make_case([300, 1, 2000], seed=32)
    note("decode counter preloaded -1")
    c = case.to(DEV)
    kp, vp = (t.to(DEV) for t in case.appended_pools())
    want = oracle_decode(case)
    S = 4
    for own_buffer in (True, False):
        if own_buffer:  # a caller-owned buffer, zeroed by the caller
            ctr = torch.zeros(2 * case.B * 2, dtype=torch.int32, device=DEV)
        else:  # the library's persistent buffer
            ctr = split_counters(torch.device(DEV), 2 * case.B * 2)
        with torch.inference_mode():  # the library's buffer may be an inference tensor
            ctr[2 * 1 + 0] = -1  # arrival word of (sequence 1, kv head 0)
        err = err_word()
        decode_gqa_attention(c.q, kp, vp, c.attended, c.slot_ids, c.block_table, num_programs=S,
                             counters=ctr if own_buffer else None, err=err)
        torch.cuda.synchronize()
        assert int(err.item()) & 8, "CIE_ERRBIT_SPLIT expected"
        if own_buffer:
            with torch.inference_mode():
                ctr.zero_()
        else:
            reset_split_counters(torch.device(DEV))
        assert torch.count_nonzero(ctr) == 0
        err.zero_()
        o = decode_gqa_attention(c.q, kp, vp, c.attended, c.slot_ids, c.block_table, num_programs=S,
                                 counters=ctr if own_buffer else None, err=err)
        torch.cuda.synchronize()
        assert int(err.item()) == 0
        assert torch.count_nonzero(ctr) == 0
        assert_attn_close(o[0].float().cpu(), want, what="call after the reset")
