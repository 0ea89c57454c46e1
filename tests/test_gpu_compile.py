"""The drop-in attention layer compiled with ``torch.compile(fullgraph=True,
backend="aot_eager")`` — Dynamo tracing plus AOT functionalization of the ops
that append to the pools, then eager execution of the traced graph (no
generated kernels) — gives the eager layer's output and pool contents bit for
bit: the fake impls, mutation annotations and op schemas are what the
reference's compiled decode step (scheduler/decode_module.py:33-44) relies on.
"""
import pytest
import torch

from tests.gpu_helpers import DEV, note
from tests.test_compile_trace import layer_step

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fuse_rope", [True, False], ids=["fused", "unfused"])
@pytest.mark.parametrize("decode", [True, False], ids=["decode", "mixed"])
def test_compiled_layer_matches_eager(native_lib, decode, fuse_rope):
    layer, kv, meta, hidden, cos, sin = layer_step(decode, DEV, seed=3)
    layer.fuse_rope = fuse_rope
    note(f"compile decode={decode} fuse_rope={fuse_rope}")
    k0, v0 = kv.keys[0].clone(), kv.values[0].clone()

    def step(h, c, s):
        return layer(h, (c, s), kv_manager=kv, metadata=meta)[0]

    with torch.no_grad():
        want = step(hidden, cos, sin)
        k_want, v_want = kv.keys[0].clone(), kv.values[0].clone()
        assert not torch.equal(k_want, k0), "the step appended nothing"
        kv.keys[0].copy_(k0)
        kv.values[0].copy_(v0)
        torch._dynamo.reset()
        got = torch.compile(step, backend="aot_eager", fullgraph=True)(hidden, cos, sin)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.equal(kv.keys[0], k_want) and torch.equal(kv.values[0], v_want)
