"""hipGraph capture (``graphs.StepGraph``) of the decode and mixed steps.

Every replay is compared bit for bit with the same step run eagerly on a
separate copy of the state, with eager work and synchronisations between
replays, and with the step's inputs changed between replays.
"""
import pytest
import torch

from custom_inference_engine_amd import decode_gqa_attention, kv_append_decode, kv_append_tokens, mixed_gqa_attention
from custom_inference_engine_amd.graphs import StepGraph
from oracle import inputs
from tests.conftest import assert_attn_close
from tests.gpu_helpers import DEV, bits, note
from oracle import paged_attention as ref

pytestmark = pytest.mark.gpu


class DecodeState:
    """Static buffers of one layer's decode step (pools, lens, inputs)."""

    def __init__(self, case):
        c = case.to(DEV)
        self.kp, self.vp = c.k_pool.clone(), c.v_pool.clone()
        self.lens = c.lens_pool.clone()
        self.slot_ids, self.bt = c.slot_ids, c.block_table
        B = case.B
        self.q, self.k_new, self.v_new = (c.q[:, :B].clone(), c.k_new[:, :B].clone(),
                                          c.v_new[:, :B].clone())

    def step(self):
        kv_append_decode(self.kp, self.vp, self.k_new, self.v_new, self.slot_ids, self.lens, self.bt)
        o = decode_gqa_attention(self.q, self.kp, self.vp, self.lens[self.slot_ids] + 1, self.slot_ids,
                                 self.bt)
        self.lens[self.slot_ids] += 1
        return o

    def restore(self, case):
        c = case.to(DEV)
        self.kp.copy_(c.k_pool)
        self.vp.copy_(c.v_pool)
        self.lens.copy_(c.lens_pool)

    def load_inputs(self, gen):
        for t in (self.q, self.k_new, self.v_new):
            t.copy_((torch.randn(t.shape, generator=gen) * 0.5).half())


def test_decode_step_graph_replays_match_eager(native_lib):
    # new_lens = 5: block tables hold pages for 5 more tokens per sequence (4 replays + warm-up
    # state is separate); only the first B new rows are used as decode inputs.
    case = inputs.make_case([100, 509, 37, 2000, 0, 15], [5] * 6, seed=41)
    note("graph decode capture")
    graph_state, eager_state = DecodeState(case), DecodeState(case)

    # the capture's warm-up ran one eager step on graph_state: put it back
    g = StepGraph(graph_state.step)
    static_out = g.output
    graph_state.restore(case)
    torch.cuda.synchronize()

    gen_g, gen_e = torch.Generator().manual_seed(5), torch.Generator().manual_seed(5)
    for i in range(4):
        note(f"graph decode replay {i}")
        graph_state.load_inputs(gen_g)
        eager_state.load_inputs(gen_e)
        g.replay()
        eager_out = eager_state.step()
        torch.cuda.synchronize()
        assert torch.equal(bits(static_out), bits(eager_out)), f"replay {i}"
        assert torch.equal(graph_state.lens, eager_state.lens)
        assert torch.equal(bits(graph_state.kp), bits(eager_state.kp))
        # eager work between replays
        _ = (eager_state.kp.float().sum() + graph_state.vp.float().sum()).item()

    # and the captured output is the right answer for the last step
    kp, vp = eager_state.kp.cpu(), eager_state.vp.cpu()
    want = ref.decode_attention(eager_state.q.cpu(), kp, vp, eager_state.lens[eager_state.slot_ids].cpu(),
                                case.slot_ids, case.block_table)
    assert_attn_close(static_out[0].float().cpu(), want, what="graph decode vs oracle")


def test_mixed_step_graph_replays_match_eager(native_lib):
    case = inputs.make_case([0, 300, 47, 1024], [64, 1, 17, 2], seed=42)
    note("graph mixed capture")
    c = case.to(DEV)

    def make():
        return {"kp": c.k_pool.clone(), "vp": c.v_pool.clone(), "q": c.q.clone(),
                "k": c.k_new.clone(), "v": c.v_new.clone()}

    def step(s):
        kv_append_tokens(s["kp"], s["vp"], s["k"], s["v"], c.pages, c.offsets)
        return mixed_gqa_attention(s["q"], s["kp"], s["vp"], 64, c.cu_seqlens, c.kv_lens, c.slot_ids,
                                   c.block_table)

    gs, es = make(), make()
    g = StepGraph(lambda: step(gs))
    static_out = g.output
    gs["kp"].copy_(c.k_pool)  # the capture's warm-up appended once
    gs["vp"].copy_(c.v_pool)
    torch.cuda.synchronize()
    gen_g, gen_e = torch.Generator().manual_seed(7), torch.Generator().manual_seed(7)
    T = case.T
    for i in range(3):
        note(f"graph mixed replay {i}")
        for s, gen in ((gs, gen_g), (es, gen_e)):
            for key in ("q", "k", "v"):
                s[key].copy_((torch.randn(s[key].shape, generator=gen) * 0.5).half())
        g.replay()
        eager_out = step(es)
        torch.cuda.synchronize()
        assert torch.equal(bits(static_out[:, :T]), bits(eager_out[:, :T])), f"replay {i}"
        assert torch.equal(bits(gs["kp"]), bits(es["kp"]))
