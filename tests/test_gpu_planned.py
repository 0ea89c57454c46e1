"""The planned decode: one plan per decode step (decode_plan), then each layer's
planned launch, against the oracle and against the unplanned launch.

A plan fixes every sequence's split count (balanced by length over the grid),
its slot and length and each workgroup's page ids; the planned kernels must
append bit-exactly, attend within the tolerance of tests/conftest.py, and give
the unplanned kernels' bits when the plan deals the same splits (equal lengths,
the same split count).  Layers of a step share one plan, graph replays of a
planned step equal the eager step, and index errors are reported by the plan.
"""
import pytest
import torch

from custom_inference_engine_amd import (decode_append_gqa_attention, decode_gqa_attention, decode_plan,
                                         decode_qkv_rope_gqa_attention)
from custom_inference_engine_amd.attn.core import split_counters
from oracle import inputs
from oracle import paged_attention as ref
from tests.conftest import assert_attn_close
from tests.gpu_helpers import DEV, bits, err_word, note, oracle_decode
from tests.test_gpu_rope import _qkv, _tables

pytestmark = pytest.mark.gpu


def _fused(case, splits=None, plan_splits=None, planned=True, err=None):
    c = case.to(DEV)
    kp, vp = c.k_pool.clone(), c.v_pool.clone()
    plan = decode_plan(kp, c.lens_pool, c.slot_ids, c.block_table, append=True, num_programs=plan_splits,
                       err=err) if planned else None
    o = decode_append_gqa_attention(c.q, kp, vp, c.k_new, c.v_new, c.lens_pool, c.slot_ids, c.block_table,
                                    num_programs=splits, err=err, plan=plan)
    torch.cuda.synchronize()
    return kp.cpu(), vp.cpu(), o[0].float().cpu()


@pytest.mark.parametrize("make,splits", [
    (lambda: inputs.config1(), None),
    (lambda: inputs.config2(seed=0), None),
    (lambda: inputs.config2(seed=3, fixed=False), None),
    (lambda: inputs.config2(seed=3, fixed=False), 16),
    (lambda: inputs.config4(), 16),
    (lambda: inputs.make_case([0, 1, 14, 15, 16, 30, 31, 32, 47, 63, 64, 127], seed=61), None),
    (lambda: inputs.make_case([0, 1, 14, 15, 16, 30, 31, 32, 47, 63, 64, 127], seed=61), 1),
    (lambda: inputs.make_case([5, 100, 333, 4000], seed=62, h_q=16, h_kv=1, d=128, page_size=32), None),
    (lambda: inputs.make_case([3000], seed=63, h_q=8, h_kv=8, page_size=64), None),
    (lambda: inputs.make_case(None, random_lens=(0, 600, 100), seed=69), None),
    (lambda: inputs.make_case(None, random_lens=(0, 300, 300), seed=70), None),
], ids=["cfg1", "cfg2", "cfg2var", "cfg2var-16", "cfg4-16", "edges", "edges-1", "g16-d128-ps32", "mha-b1",
        "b100-block-plan", "b300-block-plan"])
def test_planned_append_decode(native_lib, make, splits):
    case = make()
    note(f"planned fused decode B={case.B} splits={splits}")
    err = err_word()
    kp, vp, o = _fused(case, plan_splits=splits, err=err)
    ko, vo = case.appended_pools()
    assert torch.equal(bits(kp), bits(ko)) and torch.equal(bits(vp), bits(vo)), "append not bit-exact"
    assert_attn_close(o, oracle_decode(case), what="planned fused decode")
    assert int(err.item()) == 0


@pytest.mark.parametrize("make,splits", [
    (lambda: inputs.config2(seed=0), 4),
    (lambda: inputs.config4(), 16),
    (lambda: inputs.make_case([700] * 5, seed=64), 7),
])
def test_planned_equals_unplanned_on_equal_lengths(native_lib, make, splits):
    """Equal lengths and the same split count: the plan deals what the unplanned grid
    deals, so the outputs agree bit for bit."""
    case = make()
    note(f"planned == unplanned B={case.B} splits={splits}")
    kp1, vp1, o1 = _fused(case, splits=splits, planned=False)
    kp2, vp2, o2 = _fused(case, plan_splits=splits)
    assert torch.equal(bits(kp1), bits(kp2)) and torch.equal(bits(vp1), bits(vp2))
    assert torch.equal(o1, o2)


def test_planned_plain_decode(native_lib):
    """The plan of the plain op (append=False: lens are attended lengths per sequence)."""
    case = inputs.make_case([10, 900, 2047, 0, 4096, 33], seed=65)
    note("planned plain decode")
    c = case.to(DEV)
    kp, vp = (t.to(DEV) for t in case.appended_pools())
    lens = c.attended.clone()
    lens[3] = 0  # an empty sequence
    plan = decode_plan(kp, lens, c.slot_ids, c.block_table, append=False)
    o = decode_gqa_attention(c.q, kp, vp, lens, c.slot_ids, c.block_table, plan=plan)
    o_ref = decode_gqa_attention(c.q, kp, vp, lens, c.slot_ids, c.block_table)
    torch.cuda.synchronize()
    keep = [0, 1, 2, 4, 5]
    assert_attn_close(o[0, keep], oracle_decode(case)[keep], what="planned plain")
    assert_attn_close(o[0], o_ref[0], what="planned vs unplanned")
    assert torch.count_nonzero(o[0, 3]) == 0  # an empty sequence gives 0


def test_planned_rope_decode(native_lib):
    case = inputs.make_case(None, random_lens=(0, 3000, 19), seed=66)
    pos = case.lens_pool[case.slot_ids]
    cos, sin = _tables(pos, 64)
    q_rot = ref.rope(case.q[0], cos, sin)[None]
    k_rot = ref.rope(case.k_new[0], cos, sin)[None]
    note(f"planned rope decode B={case.B}")
    c = case.to(DEV)
    kp, vp = c.k_pool.clone(), c.v_pool.clone()
    plan = decode_plan(kp, c.lens_pool, c.slot_ids, c.block_table, append=True)
    o = decode_qkv_rope_gqa_attention(_qkv(case).to(DEV), cos[None].to(DEV), sin[None].to(DEV), kp, vp,
                                      c.lens_pool, c.slot_ids, c.block_table, num_heads=14, plan=plan)
    torch.cuda.synchronize()
    ko, vo = case.k_pool.clone(), case.v_pool.clone()
    ref.append_decode(ko, vo, k_rot, case.v_new, case.slot_ids, case.lens_pool, case.block_table)
    assert torch.equal(bits(kp.cpu()), bits(ko)) and torch.equal(bits(vp.cpu()), bits(vo))
    assert_attn_close(o[0], ref.decode_attention(q_rot, ko, vo, pos + 1, case.slot_ids, case.block_table),
                      what="planned rope decode")


def test_one_plan_serves_every_layer_and_replays(native_lib):
    """Three layers (own pools, q and new rows) of one step share a plan; recorded
    in a hipGraph with the plan launch and replayed twice, each replay equals the
    eager step bit for bit, and the split counters are left zero."""
    case = inputs.make_case(None, random_lens=(100, 4000, 24), seed=67)
    note(f"plan shared by 3 layers, graph replay B={case.B}")
    c = case.to(DEV)
    g = torch.Generator(device=DEV).manual_seed(5)

    def rnd(t):
        return (torch.randn(t.shape, generator=g, device=DEV) * 0.5).half()

    layers = [(c.k_pool.clone(), c.v_pool.clone(), c.q, c.k_new, c.v_new)]
    layers += [(rnd(c.k_pool), rnd(c.v_pool), rnd(c.q), rnd(c.k_new), rnd(c.v_new)) for _ in range(2)]
    base = [(kp.clone(), vp.clone()) for kp, vp, *_ in layers]

    def step():
        plan = decode_plan(layers[0][0], c.lens_pool, c.slot_ids, c.block_table, append=True)
        return [decode_append_gqa_attention(q, kp, vp, kn, vn, c.lens_pool, c.slot_ids, c.block_table,
                                            plan=plan) for kp, vp, q, kn, vn in layers]

    def restore():
        for (kp, vp, *_), (k0, v0) in zip(layers, base):
            kp.copy_(k0)
            vp.copy_(v0)

    eager = [o.clone() for o in step()]
    pools = [(kp.clone(), vp.clone()) for kp, vp, *_ in layers]
    torch.cuda.synchronize()
    # layer 0 against the oracle
    assert_attn_close(eager[0][0].float().cpu(), oracle_decode(case), what="layer 0")
    graph = torch.cuda.CUDAGraph()
    restore()
    torch.cuda.synchronize()
    with torch.inference_mode():
        with torch.cuda.graph(graph):
            outs = step()
    for replay in range(2):
        restore()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for li in range(3):
            assert torch.equal(outs[li], eager[li]), f"replay {replay} layer {li}"
            assert torch.equal(layers[li][0], pools[li][0]) and torch.equal(layers[li][1], pools[li][1])
    assert torch.count_nonzero(split_counters(torch.device(DEV), 2 * case.B * 2)) == 0


def test_plan_reports_index_errors(native_lib):
    """A slot id outside the table and a length past the row's capacity are reported
    by the plan (CIE_ERRBIT_PAGE, CIE_ERRBIT_LEN); the decode then skips those
    sequences (o = 0) and the others stay correct."""
    case = inputs.make_case([40, 300, 500], seed=68)
    note("plan index errors")
    c = case.to(DEV)
    kp, vp = (t.to(DEV) for t in case.appended_pools())
    slots = c.slot_ids.clone()
    slots[0] = 10_000
    lens = c.attended.clone()
    lens[1] = c.block_table.shape[1] * 16 + 5
    err = err_word()
    plan = decode_plan(kp, lens, slots, c.block_table, append=False, err=err)
    o = decode_gqa_attention(c.q, kp, vp, lens, slots, c.block_table, plan=plan, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) & 1 and int(err.item()) & 2
    assert torch.count_nonzero(o[0, 0]) == 0
    assert_attn_close(o[0, 2].float().cpu(), oracle_decode(case)[2], what="untouched sequence")
