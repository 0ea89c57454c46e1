"""The continuous-batching policy (scheduler/scheduler.py of the reference) on the CPU.

A fake step executor stands in for the GPU step modules: it checks the
invariants the kernels rely on (every fed token lands in a page the slot owns,
no page shared between slots, the pool's ``lens`` equal the scheduler's KV
lengths) and answers with a token that depends only on the request and the
position it is generated at, so results must not depend on batching or
preemption.  Expected step traces are derived by hand from the reference's
rules (scheduler.py:209-218, 377-433, 576-653).
"""
import pytest
import torch
from transformers import Qwen2Config

from custom_inference_engine_amd import KVStorage
from custom_inference_engine_amd.scheduler import Scheduler, batch_buckets, token_buckets

EOS = 999


def token_at(prompt_len: int, position: int) -> int:
    return (7 * position + 3 * prompt_len) % 50 + 1


class FakeExecutor:
    def __init__(self):
        self.sched = None
        self.trace = []

    def _check(self, slot_ids):
        s = self.sched
        kv = s.kv_cache
        owned = {}
        for slot in s.order:
            req = s.slots[slot]
            for p in req.pages:
                assert p != kv.unused_idx, "page 0 is reserved"
                assert p not in owned, f"page {p} owned by slots {owned[p]} and {slot}"
                owned[p] = slot
            row = kv.block_table[slot, :len(req.pages)].tolist()
            assert row == req.pages
            assert kv.block_table[slot, len(req.pages):].eq(0).all()
            assert int(kv.lens[slot]) == req.kv_len
        assert sum(s.slots[x].budget for x in slot_ids) <= s.token_budget
        for slot in slot_ids:
            req = s.slots[slot]
            assert req.kv_len + req.budget <= len(req.pages) * s.page_size, "tokens past the slot's pages"

    def _answer(self, slot_ids, lens):
        s = self.sched
        out = []
        for slot, n in zip(slot_ids, lens):
            req = s.slots[slot]
            s.kv_cache.lens[slot] += n
            out.append(token_at(len(req.prompt), req.kv_len + n))
        return out

    def decode(self, slot_ids):
        self._check(slot_ids)
        assert all(self.sched.slots[x].prefilled for x in slot_ids)
        self.trace.append(("decode", list(slot_ids)))
        return self._answer(slot_ids, [1] * len(slot_ids))

    def mixed(self, chunks, slot_ids):
        self._check(slot_ids)
        s = self.sched
        for slot, chunk in zip(slot_ids, chunks):
            req = s.slots[slot]
            full = req.prompt + req.new_tokens
            assert chunk == full[req.kv_len:req.kv_len + req.budget]
        self.trace.append(("mixed", list(slot_ids), [len(c) for c in chunks]))
        return self._answer(slot_ids, [len(c) for c in chunks])


def make(n_slots=4, max_cache_len=1024, budget=160, max_new=3, eos=(EOS,)):
    cfg = Qwen2Config(hidden_size=64, num_attention_heads=4, num_key_value_heads=2, num_hidden_layers=1)
    kv = KVStorage(cfg, max_cache_len=max_cache_len, page_size=16, n_slots=n_slots, device="cpu",
                   dtype=torch.float16)
    ex = FakeExecutor()
    s = Scheduler(model=None, kv_cache=kv, eos_token_ids=set(eos), max_new_tokens=max_new,
                  token_budget=budget, executor=ex)
    ex.sched = s
    return s, ex


def expected_tokens(prompt_len, max_new):
    return [token_at(prompt_len, prompt_len + i) for i in range(max_new)]


def test_buckets_follow_the_reference_rules():
    assert batch_buckets(33) == [1, 2, 4, 8, 16, 32]
    assert batch_buckets(4) == [1, 2, 4]
    assert token_buckets(512) == [16, 32, 64, 128] + list(range(160, 513, 32))


def test_chunked_prefill_budget_and_admission_trace():
    s, ex = make()
    prompts = [[5] * 100, [6] * 100, [7] * 30]
    res = s.generate(prompts)
    assert ex.trace == [
        ("mixed", [1, 2], [100, 60]),        # A whole, B gets the rest of the budget
        ("mixed", [1, 2, 3], [1, 40, 30]),   # A decodes, B finishes its prompt, C admitted
        ("decode", [1, 2, 3]),
        ("decode", [2, 3]),                  # A finished after 3 tokens
    ]
    for p, r in zip(prompts, res):
        assert r.new_tokens == expected_tokens(len(p), 3)
    assert s.stats.preemptions == 0
    assert s.stats.decode_steps == {4: 1, 2: 1}
    assert s.stats.mixed_steps == {160: 1, 128: 1}   # 160 tokens, then 71
    # everything released: all pages free again, pool rows cleared
    assert len(s._free_pages) == s.n_pages - 1
    assert s.kv_cache.lens.eq(0).all() and s.kv_cache.block_table.eq(0).all()


def test_page_aligned_chunk_takes_one_extra_page():
    s, ex = make(max_new=2)
    fut = s.call([1] * 32)
    s.stop()
    assert s.step()                     # admit + prefill the 32 tokens
    assert len(s.slots[1].pages) == 3   # ceil(33 / 16): room for the first decoded token
    assert s.slots[1].prefilled and s.slots[1].kv_len == 32
    s.loop()
    assert fut.result().new_tokens == expected_tokens(32, 2)
    assert ex.trace == [("mixed", [1], [32]), ("decode", [1])]


def test_preemption_recomputes_and_results_do_not_change():
    # 9 usable pages (144 tokens); three 40-token prompts generating 20 tokens need 12
    s, ex = make(max_cache_len=160, max_new=20)
    prompts = [[3] * 40, [4] * 40, [5] * 40]
    res = s.generate(prompts)
    for p, r in zip(prompts, res):
        assert r.new_tokens == expected_tokens(len(p), 20)
    assert s.stats.preemptions == 1
    assert s.stats.recomputed_tokens == 48     # C held 40 prompt + 8 fed tokens
    # the preempted request (the newest, slot 3) came back through a mixed step
    # that recomputed prompt + generated tokens: 40 + 9 = 49
    assert any(t[0] == "mixed" and t[2] == [49] for t in ex.trace)


def test_eos_ends_a_request_early():
    first = token_at(20, 20)
    s, ex = make(max_new=10, eos=(first,))
    res = s.generate([[1] * 20, [2] * 24])
    assert res[0].new_tokens == [first]
    assert res[1].new_tokens == expected_tokens(24, 10)[:len(res[1].new_tokens)]


def test_more_requests_than_slots_are_served_in_order():
    s, ex = make(n_slots=3, max_new=4)
    prompts = [[i + 1] * (10 + 7 * i) for i in range(7)]
    res = s.generate(prompts)
    for p, r in zip(prompts, res):
        assert r.new_tokens == expected_tokens(len(p), 4)
    assert max(len(t[1]) for t in ex.trace) <= 2


def test_call_rejects_bad_requests_and_constructor_checks():
    s, _ = make(max_cache_len=160, max_new=20)
    with pytest.raises(ValueError):
        s.call([]).result(timeout=0)
    with pytest.raises(ValueError):
        s.call([1] * 200).result(timeout=0)   # more than the pool can ever hold
    with pytest.raises(ValueError):
        make(budget=100)                      # not above the full-graph threshold
    with pytest.raises(ValueError):
        make(budget=170)                      # not a multiple of the piecewise step
    with pytest.raises(ValueError):
        make(eos=())
