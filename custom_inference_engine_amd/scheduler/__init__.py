"""Step modules and continuous batching around the attention path.

``DecodeModule`` replays a whole-model decode step from one hipGraph per batch
bucket; ``MixedModule`` / ``FullMixedModule`` / ``PiecewiseMixedModule`` run a
packed chunked-prefill / decode step eagerly, from one hipGraph per token
bucket, or compiled through the piecewise backend (hipGraph pieces between
eager varlen attention calls).  All of them take their per-step inputs as one
pinned block copied in one transfer and derive the step's metadata on the
device (``graphs.StepInputs`` / ``graphs.StepGraph``).  ``Scheduler``
(scheduler/scheduler.py of the reference) is the continuous-batching policy
around them: token budget, chunked prefill, page allocation, recompute
preemption.
"""
from .decode_module import DecodeModule  # noqa: F401
from .mixed_module import FullMixedModule, MixedModule, PiecewiseMixedModule  # noqa: F401
from .scheduler import (ModuleExecutor, Request, RequestResult, RunStats, Scheduler,  # noqa: F401
                        batch_buckets, token_buckets)
from .slots import assign_pages, pad_slot_ids  # noqa: F401
