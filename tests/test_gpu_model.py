"""A Qwen2 model through the drop-in: mixed prefill, then hipGraph-replayed decode steps.

Two layers of the Qwen2.5-0.5B layer shape (hidden 896, 14 / 2 heads, D 64) with
random weights run through ``MixedModule`` (one packed prefill step of three
prompts) and ``DecodeModule`` (a captured graph of the whole decode step for a
batch bucket of 4, one slot padded).  After every step, each sequence's logits
must match HF's own forward of the same weights in fp32 on the CPU over the
contiguous token sequence (the fallback path of attn/core.py:164-168).
"""
import copy

import pytest
import torch
from transformers import Qwen2Config, Qwen2ForCausalLM

from custom_inference_engine_amd import KVStorage, use_triton_attention
from custom_inference_engine_amd.scheduler import DecodeModule, MixedModule, assign_pages
from tests.gpu_helpers import DEV, note

pytestmark = pytest.mark.gpu


def _model():
    cfg = Qwen2Config(hidden_size=896, num_attention_heads=14, num_key_value_heads=2,
                      intermediate_size=1024, num_hidden_layers=2, vocab_size=512,
                      max_position_embeddings=4096, rope_theta=1e6, rms_norm_eps=1e-6,
                      tie_word_embeddings=True)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    ref = Qwen2ForCausalLM(cfg).float().eval()
    return cfg, ref


def _ref_logits(ref, tokens):
    with torch.no_grad():
        out = ref(input_ids=torch.tensor([tokens]), use_cache=False)
    return out.logits[0, -1]


def _rel(a, b):
    return ((a.float().cpu() - b).norm() / b.norm()).item()


def test_qwen2_model_mixed_prefill_then_graph_decode(native_lib):
    cfg, ref = _model()
    ours = copy.deepcopy(ref).half().to(DEV)
    use_triton_attention(ours)
    kv = KVStorage(cfg, max_cache_len=2048, page_size=16, n_slots=5, device=DEV, dtype=torch.float16)
    note("model decode module capture")
    dec = DecodeModule(ours, kv, batch_size=4)
    mix = MixedModule(ours, kv, token_count=128)

    g = torch.Generator().manual_seed(5)
    free = (torch.randperm(kv.n_pages - 1, generator=g) + 1).tolist()
    slots = [1, 2, 3]
    prompts = [torch.randint(0, 512, (n,), generator=g).tolist() for n in (37, 5, 20)]
    for s, p in zip(slots, prompts):
        assign_pages(kv, s, len(p) + 8, free)

    note("model mixed prefill")
    nxt = mix.forward(prompts, slots)
    seqs = [p + [t] for p, t in zip(prompts, nxt)]
    for i, p in enumerate(prompts):
        want = _ref_logits(ref, p)
        rel = _rel(mix.last_logits[i], want)
        assert rel < 2e-2, f"prefill seq {i}: rel err {rel:.3e}"

    for step in range(3):
        note(f"model graph decode {step}")
        nxt = dec.forward(slots)
        logits = dec.logits[:3].clone()
        for i in range(3):
            want = _ref_logits(ref, seqs[i])
            rel = _rel(logits[i], want)
            assert rel < 2e-2, f"decode step {step} seq {i}: rel err {rel:.3e}"
            seqs[i].append(nxt[i])
    assert kv.lens[slots].tolist() == [len(s) - 1 for s in seqs]


def test_full_mixed_module_graph_matches_eager(native_lib):
    """A prefill step replayed from FullMixedModule's graph (batch padded to 4 with the
    reserved slot, cu_seqlens padded, max_seqlen = the bucket) equals the eager step."""
    from custom_inference_engine_amd.scheduler import FullMixedModule

    cfg, ref = _model()
    ours = copy.deepcopy(ref).half().to(DEV)
    use_triton_attention(ours)
    g = torch.Generator().manual_seed(9)
    prompts = [torch.randint(0, 512, (n,), generator=g).tolist() for n in (37, 5, 20)]
    slots = [1, 2, 3]
    results = []
    for graph in (False, True):
        kv = KVStorage(cfg, max_cache_len=2048, page_size=16, n_slots=5, device=DEV, dtype=torch.float16)
        note(f"mixed module, graph={graph}")
        mod = (FullMixedModule(ours, kv, batch_size=4, token_count=64) if graph
               else MixedModule(ours, kv, token_count=64))
        free = (torch.randperm(kv.n_pages - 1, generator=torch.Generator().manual_seed(3)) + 1).tolist()
        for s, p in zip(slots, prompts):
            assign_pages(kv, s, len(p) + 8, free)
        nxt = mod.forward(prompts, slots)
        # a second, shorter step on top (decode rows through the mixed path)
        nxt2 = mod.forward([[t] for t in nxt], slots)
        torch.cuda.synchronize()
        results.append((nxt, nxt2, mod.last_logits.float().cpu(), kv.lens.cpu(), kv.keys[0].cpu()))
    (a1, a2, la, lens_a, k_a), (b1, b2, lb, lens_b, k_b) = results
    assert a1 == b1 and a2 == b2
    assert torch.equal(lens_a, lens_b) and lens_a[slots].tolist() == [len(p) + 1 for p in prompts]
    assert torch.allclose(la, lb, rtol=1e-3, atol=1e-3)
    assert torch.allclose(k_a[1:].float(), k_b[1:].float(), rtol=1e-3, atol=1e-3)  # page 0: padding


def test_piecewise_mixed_module_matches_eager(native_lib):
    """Steps through PiecewiseMixedModule (hipGraph pieces between eager varlen
    attention calls) equal the eager module's: a prefill of three prompts, decode
    rows for them, then batches of one and two sequences, all through the one
    compile of the bucket."""
    from custom_inference_engine_amd.scheduler import PiecewiseMixedModule

    cfg, ref = _model()
    ours = copy.deepcopy(ref).half().to(DEV)
    use_triton_attention(ours)
    g = torch.Generator().manual_seed(21)
    prompts = [torch.randint(0, 512, (n,), generator=g).tolist() for n in (37, 5, 20)]
    slots = [1, 2, 3]
    results = []
    for piecewise in (False, True):
        torch._dynamo.reset()
        kv = KVStorage(cfg, max_cache_len=2048, page_size=16, n_slots=5, device=DEV, dtype=torch.float16)
        note(f"mixed module, piecewise={piecewise}")
        if piecewise:
            buffer = torch.zeros((1, 64, kv.num_q_heads, kv.head_dim), dtype=torch.float16, device=DEV)
            mod = PiecewiseMixedModule(ours, kv, token_count=64, buffer=buffer,
                                       pool=torch.cuda.graph_pool_handle())
        else:
            mod = MixedModule(ours, kv, token_count=64)
        free = (torch.randperm(kv.n_pages - 1, generator=torch.Generator().manual_seed(3)) + 1).tolist()
        for s, p in zip(slots, prompts):
            assign_pages(kv, s, len(p) + 8, free)
        steps = [mod.forward(prompts, slots)]
        logits = [mod.last_logits.float().cpu()]
        steps.append(mod.forward([[t] for t in steps[-1]], slots))
        logits.append(mod.last_logits.float().cpu())
        steps.append(mod.forward([[steps[-1][1], 7, 9]], [2]))
        logits.append(mod.last_logits.float().cpu())
        steps.append(mod.forward([[steps[-2][0]], [steps[-2][2], 3]], [1, 3]))
        logits.append(mod.last_logits.float().cpu())
        torch.cuda.synchronize()
        if piecewise:
            # one compile (fixed shapes), and every step replayed its recorded pieces
            # (3 per step for 2 layers) instead of falling back to eager
            assert mod.backend.compiles == 1
            assert mod.backend.piece_replays >= 4 * 3
        results.append((steps, logits, kv.lens.cpu(), torch.stack(kv.keys).cpu(), torch.stack(kv.values).cpu()))
    (sa, la, lens_a, k_a, v_a), (sb, lb, lens_b, k_b, v_b) = results
    assert sa == sb
    assert torch.equal(lens_a, lens_b)
    assert lens_a[slots].tolist() == [len(p) + d for p, d in zip(prompts, (2, 4, 3))]
    for x, y in zip(la, lb):
        assert torch.allclose(x, y, rtol=1e-3, atol=1e-3)
    # page 0 holds the padding tokens' appends
    assert torch.allclose(k_a[:, 1:].float(), k_b[:, 1:].float(), rtol=1e-3, atol=1e-3)
    assert torch.allclose(v_a[:, 1:].float(), v_b[:, 1:].float(), rtol=1e-3, atol=1e-3)
