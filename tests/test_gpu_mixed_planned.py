"""Planned mixed attention: one plan per mixed step (cie_mixed_plan), read by
every layer's launch (cie_mixed_attention_planned).

A planned launch runs the same work items, in the same order, with the same
partial bases as the unplanned launch plans for itself, so its output must
equal the unplanned output bit for bit (and the oracle within tolerance).
"""
import pytest
import torch

from custom_inference_engine_amd import _native, mixed_gqa_attention, mixed_plan
from oracle import inputs
from tests.conftest import assert_attn_close
from tests.gpu_helpers import DEV, err_word, note, oracle_mixed

pytestmark = pytest.mark.gpu


def _both(case, max_seqlen=None, partials_bytes=None):
    """(unplanned o, planned o, plan err word) for one case on its appended pools."""
    c = case.to(DEV)
    kp, vp = (t.to(DEV) for t in case.appended_pools())
    ms = int(case.new_lens.max()) if max_seqlen is None else max_seqlen
    h_q = case.q.shape[2]
    err = err_word()
    plan = mixed_plan(kp, c.cu_seqlens, c.kv_lens, c.slot_ids, c.block_table, ms, case.T, h_q,
                      partials_bytes=partials_bytes, err=err)
    o_u = mixed_gqa_attention(c.q, kp, vp, ms, c.cu_seqlens, c.kv_lens, c.slot_ids, c.block_table,
                              partials_bytes=partials_bytes)
    # the planned call never reads cu_seqlens / kv_lens / slot_ids: pass zeros
    z = torch.zeros_like(c.kv_lens)
    o_p = mixed_gqa_attention(c.q, kp, vp, ms, torch.zeros_like(c.cu_seqlens), z, z, c.block_table,
                              partials_bytes=partials_bytes, plan=plan, err=err)
    torch.cuda.synchronize()
    return o_u[0].float().cpu(), o_p[0].float().cpu(), int(err.item())


CASES = {
    "config3": lambda: inputs.config3(),
    "shapes": lambda: inputs.make_case([0, 0, 5, 700, 16, 2000, 100, 0], [1, 17, 1, 1, 2, 1, 40, 129], seed=81),
    "long-prefixes": lambda: inputs.make_case([16000, 5, 30000, 9000], [20, 1, 1, 33], seed=82),
    "d128": lambda: inputs.make_case([5000, 3000, 0], [1, 33, 64], seed=83, d=128),
    "g8-ps32": lambda: inputs.make_case([0, 40, 300], [37, 1, 20], seed=84, h_q=8, h_kv=1, page_size=32),
    "b90-block-plan": lambda: inputs.make_case(
        [int(x) for x in torch.randint(0, 2500, (90,), generator=torch.Generator().manual_seed(85))],
        [1 + (i % 9 == 0) * 39 for i in range(90)], seed=85),
}


@pytest.mark.parametrize("name", list(CASES))
def test_planned_mixed_equals_unplanned(native_lib, name):
    case = CASES[name]()
    note(f"planned mixed {name} B={case.B} T={case.T}")
    ms = case.meta.get("max_seqlen") if name == "config3" else None
    o_u, o_p, err = _both(case, max_seqlen=ms)
    assert err == 0
    want, written = oracle_mixed(case)
    assert torch.equal(o_p[written], o_u[written]), "planned != unplanned"
    assert_attn_close(o_p[written], want[written], what=f"planned {name}")


@pytest.mark.parametrize("budget_rows", [0, 14 * 16, None])
def test_planned_mixed_partials_budgets(native_lib, budget_rows):
    """The plan carries the partial bases of its budget: no budget, one that
    splits only part of the batch, and the default."""
    case = inputs.make_case([9000, 700, 3000, 20000], [20, 1, 2, 1], seed=86)
    nbytes = None if budget_rows is None else (0 if budget_rows == 0 else 768 + budget_rows * 4 * 66)
    note(f"planned mixed budget {budget_rows} rows")
    o_u, o_p, err = _both(case, partials_bytes=nbytes)
    assert err == 0
    want, written = oracle_mixed(case)
    assert torch.equal(o_p[written], o_u[written])
    assert_attn_close(o_p[written], want[written], what=f"planned, budget {budget_rows}")


def test_one_mixed_plan_serves_every_layer_and_replays(native_lib):
    """One plan, three layers' pools and queries, recorded in a hipGraph with
    the plan kernel and replayed twice: every replay equals the unplanned
    eager calls bit for bit."""
    from custom_inference_engine_amd.graphs import StepGraph

    case = inputs.make_case([0, 256, 1500, 31, 3000], [64, 16, 1, 1, 1], seed=87)
    c = case.to(DEV)
    kp0, vp0 = (t.to(DEV) for t in case.appended_pools())
    g = torch.Generator(device=DEV).manual_seed(88)
    layers = [(kp0, vp0, c.q)] + [
        (torch.randn(kp0.shape, generator=g, device=DEV).half(), torch.randn(vp0.shape, generator=g, device=DEV).half(),
         torch.randn(c.q.shape, generator=g, device=DEV).half()) for _ in range(2)]
    ms = int(case.new_lens.max())
    h_q = case.q.shape[2]
    want = [mixed_gqa_attention(q, kp, vp, ms, c.cu_seqlens, c.kv_lens, c.slot_ids, c.block_table)
            for kp, vp, q in layers]
    torch.cuda.synchronize()
    outs = [None] * len(layers)

    def step():
        plan = mixed_plan(kp0, c.cu_seqlens, c.kv_lens, c.slot_ids, c.block_table, ms, case.T, h_q)
        for i, (kp, vp, q) in enumerate(layers):
            outs[i] = mixed_gqa_attention(q, kp, vp, ms, c.cu_seqlens, c.kv_lens, c.slot_ids, c.block_table,
                                          plan=plan)

    note("planned mixed graph: plan + 3 layers")
    graph = StepGraph(step)
    for rep in range(2):
        graph.replay()
        torch.cuda.synchronize()
        _, written = oracle_mixed(case)
        for i in range(len(layers)):
            assert torch.equal(outs[i][0].cpu()[written], want[i][0].cpu()[written]), (rep, i)
        # eager work of the program's own between the replays
        again = mixed_gqa_attention(c.q, kp0, vp0, ms, c.cu_seqlens, c.kv_lens, c.slot_ids, c.block_table)
        torch.cuda.synchronize()
        assert torch.equal(again[0].cpu()[written], want[0][0].cpu()[written])


def test_mixed_plan_for_another_batch_is_refused(native_lib):
    """A planned call whose batch shape or partials budget differs from its
    plan's writes nothing and raises CIE_ERRBIT_PLAN (16); the host refuses
    a plan buffer smaller than cie_mixed_plan_bytes."""
    case = inputs.make_case([100, 2000, 3000], [5, 1, 1], seed=89)
    c = case.to(DEV)
    kp, vp = (t.to(DEV) for t in case.appended_pools())
    lib = _native.load()
    plan = mixed_plan(kp, c.cu_seqlens, c.kv_lens, c.slot_ids, c.block_table, 5, case.T, 14)
    for what, kw in (("another budget", dict(partials_bytes=0)), ("another max_seqlen", dict(ms=40))):
        note(f"planned mixed mismatch: {what}")
        err = err_word()
        ms = kw.pop("ms", 5)
        o = mixed_gqa_attention(c.q, kp, vp, ms, c.cu_seqlens, c.kv_lens, c.slot_ids, c.block_table, plan=plan,
                                err=err, **kw)
        torch.cuda.synchronize()
        assert int(err.item()) & 16, what
    with pytest.raises(AssertionError):
        mixed_gqa_attention(c.q, kp, vp, 5, c.cu_seqlens, c.kv_lens, c.slot_ids, c.block_table,
                            plan=plan[: plan.numel() // 2])
    assert lib.cie_mixed_plan_bytes(3, case.T) <= plan.numel() * 4


def test_mixed_plan_reports_rows_past_max_seqlen(native_lib):
    """Rows past max_seqlen are not computed; the plan reports them (CIE_ERRBIT_LEN)."""
    case = inputs.make_case([0, 10], [40, 1], seed=90)
    c = case.to(DEV)
    kp, vp = (t.to(DEV) for t in case.appended_pools())
    err = err_word()
    note("mixed plan with rows past max_seqlen")
    mixed_plan(kp, c.cu_seqlens, c.kv_lens, c.slot_ids, c.block_table, 16, case.T, 14, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) & 2
