"""The TritonQwen2Attention drop-in on the GPU against HF Qwen2Attention (fp32, CPU).

A prompt goes through the mixed path (token-mode append + varlen attention),
then two decode steps go through the decode path, all on a shuffled paged
pool; each output must match HF's own attention over the contiguous sequence
(the fallback path of attn/core.py:164-168) run in fp32.
"""
import copy

import pytest
import torch
from transformers import Qwen2Config
from transformers.models.qwen2.modeling_qwen2 import Qwen2Attention, Qwen2RotaryEmbedding

from custom_inference_engine_amd import AttentionMetadata, KVStorage, TritonQwen2Attention
from oracle import paged_attention as ref
from tests.gpu_helpers import DEV, note

pytestmark = pytest.mark.gpu


def _config():
    cfg = Qwen2Config(hidden_size=896, num_attention_heads=14, num_key_value_heads=2,
                      intermediate_size=4864, num_hidden_layers=2, vocab_size=1024,
                      max_position_embeddings=4096, rope_theta=1e6)
    cfg._attn_implementation = "sdpa"
    return cfg


def _hf_attention(attn32, rope32, hidden32, positions):
    pos = torch.tensor([positions])
    emb = rope32(hidden32, pos)
    out, _ = attn32(hidden32, emb, None)
    return out


@pytest.mark.parametrize("fuse_rope,fuse_append", [(True, True), (False, True), (False, False)])
def test_qwen2_attention_dropin_prefill_then_decode(native_lib, fuse_rope, fuse_append):
    torch.manual_seed(0)
    cfg = _config()
    attn_ref = Qwen2Attention(cfg, layer_idx=1).float()
    with torch.no_grad():
        for p in attn_ref.parameters():
            p.normal_(0, 0.05)
    rope32 = Qwen2RotaryEmbedding(cfg)
    ours = TritonQwen2Attention(copy.deepcopy(attn_ref).half().to(DEV)).to(DEV)
    ours.fuse_rope, ours.fuse_append = fuse_rope, fuse_append
    rope16 = Qwen2RotaryEmbedding(cfg, device=DEV)

    kv = KVStorage(cfg, max_cache_len=1024, page_size=16, n_slots=4, device=DEV, dtype=torch.float16)
    slot = 2
    pages = torch.randperm(kv.n_pages - 1, generator=torch.Generator().manual_seed(3))[:8] + 1
    kv.block_table[slot, :8] = pages.to(DEV)

    L0 = 45
    hidden = torch.randn(1, L0 + 2, 896) * 0.5
    # prefill through the mixed path
    note("module prefill")
    meta = AttentionMetadata(token_count=L0, full_decode=False, device=DEV)
    meta.slot_ids = torch.tensor([slot], device=DEV)
    meta.cu_seqlens = torch.tensor([0, L0], device=DEV)
    pos = torch.arange(L0)
    meta.write_pages(kv.block_table[slot].cpu()[pos // 16])
    meta.write_offsets(pos % 16)
    h16 = hidden[:, :L0].half().to(DEV)
    emb = rope16(h16, pos[None].to(DEV))
    with torch.no_grad():
        out, _ = ours(h16, emb, kv_manager=kv, metadata=meta)
        kv.mixed_advance(meta.slot_ids, torch.tensor([L0], device=DEV))
        want = _hf_attention(attn_ref, rope32, hidden[:, :L0], list(range(L0)))
    torch.cuda.synchronize()
    rel = (out.float().cpu() - want).norm() / want.norm()
    assert rel < 1e-2, f"prefill rel err {rel:.3e}"

    # two decode steps through the decode path
    for step in range(2):
        note(f"module decode {step}")
        n = L0 + step
        meta_d = AttentionMetadata(token_count=1, full_decode=True, device=DEV)
        meta_d.prepare_full_graph(1)
        meta_d.write_slot_ids([slot])
        h = hidden[:, n:n + 1].half().to(DEV)
        emb = rope16(h, torch.tensor([[n]], device=DEV))
        with torch.no_grad():
            out, _ = ours(h, emb, kv_manager=kv, metadata=meta_d)
            kv.decode_advance(meta_d.slot_ids)
            full = _hf_attention(attn_ref, rope32, hidden[:, :n + 1], list(range(n + 1)))
        torch.cuda.synchronize()
        want = full[:, n:n + 1]
        rel = (out.float().cpu() - want).norm() / want.norm()
        assert rel < 1e-2, f"decode step {step} rel err {rel:.3e}"
    assert int(kv.lens[slot]) == L0 + 2
