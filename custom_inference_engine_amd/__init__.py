"""MI355X (gfx950) paged-KV GQA attention hot path with the reference engine's surface.

Modules mirror the reference's layout: ``kv_cache.storage`` (KVStorage),
``attn.metadata`` (AttentionMetadata) and ``attn.core`` (decode / mixed
attention host functions, the ``inference::*`` ops and the Qwen2 drop-in).
The kernels live in ``libcie_paged.so`` (``csrc/``, C ABI in
``include/cie_paged_attention.h``), built by ``_build.build()``.
"""
from .attn.core import (  # noqa: F401
    GQA_DECODE_CONFIG,
    GQA_PREFILL_CONFIG,
    HipQwen2Attention,
    TritonQwen2Attention,
    append_tokens_qkv_rope,
    decode_append_gqa_attention,
    decode_gqa_attention,
    decode_plan,
    decode_qkv_rope_gqa_attention,
    gqa_decode_append_attention_op,
    gqa_decode_attention_op,
    gqa_decode_plan_op,
    gqa_decode_qkv_rope_attention_op,
    gqa_mixed_attention_op,
    gqa_mixed_plan_op,
    kv_append_tokens_qkv_rope_op,
    mixed_gqa_attention,
    mixed_plan,
    replace_attention,
    reset_split_counters,
    use_triton_attention,
)
from .attn.metadata import AttentionMetadata  # noqa: F401
from .kv_cache.storage import KVStorage, kv_append_decode, kv_append_tokens  # noqa: F401
