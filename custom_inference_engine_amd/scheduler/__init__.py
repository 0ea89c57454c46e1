"""Step modules around the attention path, mirroring the reference's scheduler/ layout.

``DecodeModule`` (scheduler/decode_module.py:8-107 of the reference) captures a
whole decode step of the model — every layer's fused KV append + paged decode —
in one hipGraph per batch bucket and replays it; ``MixedModule``
(scheduler/mixed_module.py:10-133) runs a packed chunked-prefill / decode
step eagerly and ``FullMixedModule`` (scheduler/mixed_module.py:164-213)
replays it from a hipGraph per token bucket; ``PiecewiseMixedModule``
(scheduler/mixed_module.py:216-249) compiles it through the piecewise backend
(hipGraph pieces between eager varlen attention calls); ``Scheduler`` (scheduler/scheduler.py) is the continuous-batching
policy around them (token budget, chunked prefill, page allocation, recompute
preemption).
"""
from .decode_module import DecodeModule  # noqa: F401
from .mixed_module import FullMixedModule, MixedModule, PiecewiseMixedModule  # noqa: F401
from .scheduler import (ModuleExecutor, Request, RequestResult, RunStats, Scheduler,  # noqa: F401
                        batch_buckets, token_buckets)
from .slots import assign_pages, pad_slot_ids  # noqa: F401
