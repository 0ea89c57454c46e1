"""The allocation-free decode entry point (cie_paged_decode_append_noalloc) through the C ABI.

Its split partials and arrival counters live in the library's static device
array instead of caller buffers.  Two calls in a row — the second with a
smaller batch and shorter sequences, so it runs on what the first left in the
array — must each give exactly what cie_paged_decode_append gives with
caller-owned workspace (same kernels, same split count: the output and the
appended pools bit for bit), and both must match the fp32 oracle.  A problem
larger than the static array is refused with CIE_ESCRATCH before anything is
launched.
"""
import pytest
import torch

from custom_inference_engine_amd import _native
from oracle import inputs
from tests.conftest import assert_attn_close
from tests.gpu_helpers import DEV, bits, err_word, note, oracle_decode

pytestmark = pytest.mark.gpu

CIE_ESCRATCH = -3


def _args(case, c, kp, vp, o):
    rows_k = c.k_new[0]
    rows_v = c.v_new[0]
    bt = c.block_table
    return dict(
        head=(o.data_ptr(), c.q.data_ptr(), kp.data_ptr(), vp.data_ptr(), rows_k.data_ptr(),
              rows_v.data_ptr(), rows_k.stride(0), rows_k.stride(1), rows_v.stride(0), rows_v.stride(1),
              c.lens_pool.data_ptr(), c.slot_ids.data_ptr(), bt.data_ptr()),
        tail=(case.B, 14, 2, 64, 16, kp.shape[0], kp.stride(0), kp.stride(1), bt.stride(0), bt.shape[1],
              c.lens_pool.shape[0]),
    )


def _run(case, splits, noalloc: bool):
    lib = _native.load()
    c = case.to(DEV)
    kp, vp = c.k_pool.clone(), c.v_pool.clone()
    o = torch.full_like(c.q, 3.0)
    a = _args(case, c, kp, vp, o)
    err = err_word()
    stream = _native.stream_handle(torch.device(DEV))
    if noalloc:
        rc = lib.cie_paged_decode_append_noalloc(*a["head"], *a["tail"], splits, err.data_ptr(), stream)
    else:
        ws = torch.empty(lib.cie_paged_decode_partials_bytes(case.B, 14, 64, splits), dtype=torch.uint8,
                         device=DEV)
        ctr = torch.zeros(2 * case.B * 2, dtype=torch.int32, device=DEV)
        rc = lib.cie_paged_decode_append(*a["head"], ws.data_ptr(), ctr.data_ptr(), *a["tail"], splits,
                                         err.data_ptr(), stream)
    assert rc == 0, rc
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    return kp.cpu(), vp.cpu(), o[0].float().cpu()


def test_noalloc_first_call_under_graph_capture(native_lib):
    """The first call of the process (scratch address lookup and the counters' fill
    kernel included) recorded into a hipGraph, then replayed twice: each replay
    appends the new rows once and gives exactly what the workspace entry point
    gives eagerly.  Placed first: no earlier test in the run calls this entry point."""
    lib = _native.load()
    case = inputs.make_case([4095, 17, 900, 2500, 0, 1300, 64, 3000], seed=54)
    splits = 4
    note(f"noalloc under capture B={case.B} splits={splits}")
    k_ref, v_ref, o_ref = _run(case, splits, noalloc=False)
    c = case.to(DEV)
    kp, vp = c.k_pool.clone(), c.v_pool.clone()
    o = torch.full_like(c.q, 3.0)
    err = err_word()
    a = _args(case, c, kp, vp, o)
    g = torch.cuda.CUDAGraph()
    rcs = []
    # captures run in inference mode, as the package's StepGraph does (torch's
    # generator capture state, once created there, cannot be used outside it)
    with torch.inference_mode(), torch.cuda.graph(g):
        stream = _native.stream_handle(torch.device(DEV))
        rcs.append(lib.cie_paged_decode_append_noalloc(*a["head"], *a["tail"], splits, err.data_ptr(),
                                                        stream))
    assert rcs == [0], rcs
    for replay in range(2):
        kp.copy_(c.k_pool)
        vp.copy_(c.v_pool)
        o.fill_(3.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert int(err.item()) == 0
        assert torch.equal(bits(kp.cpu()), bits(k_ref)) and torch.equal(bits(vp.cpu()), bits(v_ref)), replay
        assert torch.equal(o[0].float().cpu(), o_ref), f"replay {replay} differs from the workspace entry point"
        # the rows were appended where decode_update puts them, and nowhere else
        ko, vo = case.appended_pools()
        assert torch.equal(bits(kp.cpu()), bits(ko)) and torch.equal(bits(vp.cpu()), bits(vo))


@pytest.mark.parametrize("splits", [4, 16])
def test_noalloc_matches_workspace_entry_point(native_lib, splits):
    first = inputs.make_case([4095, 17, 900, 2500, 0, 1300, 64, 3000], seed=51)
    second = inputs.make_case([700, 5, 129], seed=52)  # smaller batch, shorter sequences
    for name, case in (("first", first), ("second", second)):
        note(f"noalloc decode {name} B={case.B} splits={splits}")
        k_ref, v_ref, o_ref = _run(case, splits, noalloc=False)
        k_na, v_na, o_na = _run(case, splits, noalloc=True)
        assert torch.equal(bits(k_na), bits(k_ref)) and torch.equal(bits(v_na), bits(v_ref)), name
        assert torch.equal(o_na, o_ref), f"{name}: output differs from the workspace entry point"
        ko, vo = case.appended_pools()
        assert torch.equal(bits(k_na), bits(ko)) and torch.equal(bits(v_na), bits(vo))
        assert_attn_close(o_na, oracle_decode(case), what=f"noalloc {name}")


def test_noalloc_refuses_problems_beyond_its_scratch(native_lib):
    lib = _native.load()
    limit = lib.cie_paged_decode_noalloc_limit(14, 2, 64, 16)
    assert 0 < limit < 4096
    assert lib.cie_paged_decode_partials_bytes(limit, 14, 64, 16) <= 4 << 20
    assert lib.cie_paged_decode_partials_bytes(limit + 1, 14, 64, 16) > 4 << 20
    case = inputs.make_case([10] * (limit + 1), seed=53)
    c = case.to(DEV)
    kp, vp = c.k_pool.clone(), c.v_pool.clone()
    o = torch.full_like(c.q, 3.0)
    a = _args(case, c, kp, vp, o)
    note(f"noalloc refusal B={case.B}")
    rc = lib.cie_paged_decode_append_noalloc(*a["head"], *a["tail"], 16, None,
                                             _native.stream_handle(torch.device(DEV)))
    torch.cuda.synchronize()
    assert rc == CIE_ESCRATCH
    assert b"static scratch" in lib.cie_status_string(rc)
    assert torch.all(o == 3.0) and torch.equal(kp, c.k_pool)  # nothing ran
