"""The continuous-batching Scheduler on the GPU: a small Qwen2 served end to end.

Five prompts share three slots and a pool too small for all of them at once,
so the run admits requests as others finish, chunks prefills under the token
budget, mixes decode rows into prefill steps, and preempts (recomputes) the
newest requests twice (the policy trace is independent of the tokens, and the
CPU policy test shows these numbers for this shape).  Every generated token
must be HF's fp32 greedy choice on the same sequence, up to the fp16 path's
logit error (a token within 2 % of the logit range of the best one).
"""
import copy

import pytest
import torch
from transformers import Qwen2Config, Qwen2ForCausalLM

from custom_inference_engine_amd import KVStorage, use_triton_attention
from custom_inference_engine_amd.scheduler import FullMixedModule, PiecewiseMixedModule, Scheduler
from tests.gpu_helpers import DEV, note

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("piecewise", [False, True], ids=["full_graphs", "piecewise_above_128"])
def test_scheduler_serves_prompts_with_preemption(native_lib, piecewise):
    """``piecewise``: token buckets above 128 run through ``PiecewiseMixedModule``,
    as in the reference's scheduler (scheduler/scheduler.py:157-200)."""
    torch._dynamo.reset()
    cfg = Qwen2Config(hidden_size=896, num_attention_heads=14, num_key_value_heads=2,
                      intermediate_size=1024, num_hidden_layers=2, vocab_size=512,
                      max_position_embeddings=4096, rope_theta=1e6, rms_norm_eps=1e-6,
                      tie_word_embeddings=True)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    ref = Qwen2ForCausalLM(cfg).float().eval()
    ours = copy.deepcopy(ref).half().to(DEV)
    use_triton_attention(ours)
    kv = KVStorage(cfg, max_cache_len=192, page_size=16, n_slots=4, device=DEV, dtype=torch.float16)
    note("scheduler: capturing decode buckets")
    sched = Scheduler(ours, kv, eos_token_ids={cfg.vocab_size}, max_new_tokens=16, token_budget=160,
                      piecewise_mixed=piecewise)

    g = torch.Generator().manual_seed(11)
    prompts = [torch.randint(0, cfg.vocab_size, (n,), generator=g).tolist() for n in (60, 70, 50, 9, 64)]
    note("scheduler: generate")
    with torch.inference_mode():
        results = sched.generate(prompts)
    torch.cuda.synchronize()
    assert sched.stats.preemptions == 2
    assert sched.stats.mixed_steps and sched.stats.decode_steps
    assert sched.stats.mixed_steps[160] > 0  # the bucket above 128 ran
    kind = PiecewiseMixedModule if piecewise else FullMixedModule
    assert type(sched.executor.mixed_module(160)) is kind

    for i, (p, r) in enumerate(zip(prompts, results)):
        assert len(r.new_tokens) == 16
        seq = p + r.new_tokens
        with torch.no_grad():
            logits = ref(input_ids=torch.tensor([seq[:-1]]), use_cache=False).logits[0]
        for j, tok in enumerate(r.new_tokens):
            row = logits[len(p) - 1 + j]
            margin = float(row.max() - row[tok])
            assert margin <= 2e-2 * float(row.max() - row.min()), \
                f"request {i} token {j}: {tok} is {margin:.4f} below the best logit"
    # all slots and pages released; the pool forgot every sequence
    assert kv.lens.eq(0).all() and kv.block_table.eq(0).all()


def test_scheduler_piecewise_buckets_stay_compiled(native_lib):
    """With a 224-token budget the buckets above 128 (160, 192, 224) run through
    PiecewiseMixedModule; several of them serve steps, and each compiled exactly
    once and replayed its recorded pieces on every step it served (no eager
    fallback after the constructors' compiles)."""
    torch._dynamo.reset()
    cfg = Qwen2Config(hidden_size=896, num_attention_heads=14, num_key_value_heads=2,
                      intermediate_size=1024, num_hidden_layers=2, vocab_size=512,
                      max_position_embeddings=4096, rope_theta=1e6, rms_norm_eps=1e-6,
                      tie_word_embeddings=True)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    ref = Qwen2ForCausalLM(cfg).float().eval()
    ours = copy.deepcopy(ref).half().to(DEV)
    use_triton_attention(ours)
    kv = KVStorage(cfg, max_cache_len=1024, page_size=16, n_slots=4, device=DEV, dtype=torch.float16)
    note("scheduler: piecewise buckets")
    sched = Scheduler(ours, kv, eos_token_ids={cfg.vocab_size}, max_new_tokens=4, token_budget=224,
                      piecewise_mixed=True)
    g = torch.Generator().manual_seed(12)
    prompts = [torch.randint(0, cfg.vocab_size, (n,), generator=g).tolist()
               for n in (150, 20, 10, 140, 60, 20)]  # mixed steps of 180 and 220 tokens
    with torch.inference_mode():
        results = sched.generate(prompts)
    torch.cuda.synchronize()
    served = {t: n for t, n in sched.stats.mixed_steps.items() if t > 128}
    assert len(served) >= 2, sched.stats.mixed_steps
    for t, n in served.items():
        mod = sched.executor.mixed_modules[t]
        assert type(mod) is PiecewiseMixedModule
        assert mod.backend.compiles == 1, (t, mod.backend.compiles)
        # warm-up plus n steps, each replaying the 3 recorded pieces of a 2-layer stack
        assert mod.backend.piece_replays == 3 * (n + 1), (t, n, mod.backend.piece_replays)
    for p, r in zip(prompts, results):
        assert len(r.new_tokens) == 4
        seq = p + r.new_tokens
        with torch.no_grad():
            logits = ref(input_ids=torch.tensor([seq[:-1]]), use_cache=False).logits[0]
        for j, tok in enumerate(r.new_tokens):
            row = logits[len(p) - 1 + j]
            assert float(row.max() - row[tok]) <= 2e-2 * float(row.max() - row.min())
    assert kv.lens.eq(0).all() and kv.block_table.eq(0).all()
