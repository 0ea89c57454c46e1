"""KV append on the GPU: bit-exact against the oracle's index scatter."""
import pytest
import torch

from custom_inference_engine_amd import kv_append_decode, kv_append_tokens
from oracle import inputs, paged_attention as ref
from tests.gpu_helpers import DEV, bits, err_word, note

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("make", [
    lambda: inputs.config1(),
    lambda: inputs.config2(seed=1, fixed=False),
    lambda: inputs.make_case([0, 1, 14, 15, 16, 31, 47, 100], seed=5),
    lambda: inputs.make_case([5, 70], seed=6, page_size=32),
], ids=["config1", "config2-var", "edges", "page32"])
def test_decode_append_bit_exact(native_lib, make):
    case = make()
    note(f"decode append B={case.B}")
    c = case.to(DEV)
    kp, vp = c.k_pool.clone(), c.v_pool.clone()
    err = err_word()
    kv_append_decode(kp, vp, c.k_new, c.v_new, c.slot_ids, c.lens_pool, c.block_table, err=err)
    ko, vo = case.k_pool.clone(), case.v_pool.clone()
    ref.append_decode(ko, vo, case.k_new, case.v_new, case.slot_ids, case.lens_pool, case.block_table)
    assert torch.equal(bits(kp), bits(ko))
    assert torch.equal(bits(vp), bits(vo))
    assert int(err.item()) == 0


def test_decode_append_strided_inputs(native_lib):
    """V straight out of a fused QKV projection: token stride 1152, not 128."""
    case = inputs.make_case([3, 17, 40], seed=7)
    note("decode append strided")
    fused = torch.randn(1, case.B, 1152, generator=torch.Generator().manual_seed(0)).half()
    k_new = fused[..., 896:1024].view(1, case.B, 2, 64)
    v_new = fused[..., 1024:].view(1, case.B, 2, 64)
    assert not v_new.is_contiguous()
    c = case.to(DEV)
    fused_d = fused.to(DEV)
    kp, vp = c.k_pool.clone(), c.v_pool.clone()
    kv_append_decode(kp, vp, fused_d[..., 896:1024].view(1, case.B, 2, 64),
                     fused_d[..., 1024:].view(1, case.B, 2, 64), c.slot_ids, c.lens_pool, c.block_table)
    ko, vo = case.k_pool.clone(), case.v_pool.clone()
    ref.append_decode(ko, vo, k_new.contiguous(), v_new.contiguous(), case.slot_ids, case.lens_pool,
                      case.block_table)
    assert torch.equal(bits(kp), bits(ko)) and torch.equal(bits(vp), bits(vo))


def test_decode_append_padding_rows(native_lib):
    """Padded batch (slot 0 rows): real rows exact; padding only ever touches page 0."""
    case = inputs.make_case([9, 33], seed=8)
    note("decode append padding")
    slot_ids = torch.tensor([1, 2, 0, 0])
    k_new = torch.randn(1, 4, 2, 64, generator=torch.Generator().manual_seed(1)).half()
    c = case.to(DEV)
    kp, vp = c.k_pool.clone(), c.v_pool.clone()
    kv_append_decode(kp, vp, k_new.to(DEV), k_new.to(DEV), slot_ids.to(DEV), c.lens_pool, c.block_table)
    ko, vo = case.k_pool.clone(), case.v_pool.clone()
    ref.append_decode(ko, vo, k_new, k_new, slot_ids, case.lens_pool, case.block_table)
    assert torch.equal(bits(kp)[1:], bits(ko)[1:]) and torch.equal(bits(vp)[1:], bits(vo)[1:])
    # page 0 row 0 holds one of the padding rows (order-dependent winner, like index_put_)
    row = bits(kp)[0, :, 0]
    cands = [bits(k_new[0, i]) for i in (2, 3)]
    assert any(torch.equal(row, cnd) for cnd in cands)


@pytest.mark.parametrize("make", [
    lambda: inputs.config3(),
    lambda: inputs.make_case([0, 5, 20, 37, 0], [17, 1, 3, 1, 0], seed=3),
], ids=["config3", "mixed_small"])
def test_token_append_bit_exact(native_lib, make):
    case = make()
    note(f"token append T={case.T}")
    c = case.to(DEV)
    kp, vp = c.k_pool.clone(), c.v_pool.clone()
    err = err_word()
    kv_append_tokens(kp, vp, c.k_new, c.v_new, c.pages, c.offsets, err=err)
    ko, vo = case.appended_pools()
    assert torch.equal(bits(kp), bits(ko)) and torch.equal(bits(vp), bits(vo))
    assert int(err.item()) == 0


def test_append_out_of_range_index_is_flagged_not_written(native_lib):
    """Bad page ids / slots are skipped and reported through the error word."""
    case = inputs.make_case([4, 20], seed=9)
    note("append error flag")
    c = case.to(DEV)
    bt = c.block_table.clone()
    bt[1, 0] = case.k_pool.shape[0] + 5  # slot 1 appends at pos 4 -> logical page 0
    kp, vp = c.k_pool.clone(), c.v_pool.clone()
    err = err_word()
    kv_append_decode(kp, vp, c.k_new, c.v_new, c.slot_ids, c.lens_pool, bt, err=err)
    assert int(err.item()) & 1
    ko, vo = case.k_pool.clone(), case.v_pool.clone()
    # only slot 2's row was written
    ref.append_decode(ko, vo, case.k_new[:, 1:], case.v_new[:, 1:], case.slot_ids[1:], case.lens_pool,
                      case.block_table)
    assert torch.equal(bits(kp), bits(ko))
    # token mode: offset outside the page
    err.zero_()
    kv_append_tokens(kp, vp, c.k_new, c.v_new, c.pages[:2], torch.tensor([3, 16], device=DEV), err=err)
    assert int(err.item()) & 4
