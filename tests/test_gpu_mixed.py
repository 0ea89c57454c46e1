"""Varlen mixed (chunked prefill + decode) causal attention on the GPU against the fp32 oracle."""
import json
import os

import numpy as np
import pytest
import torch

from custom_inference_engine_amd import _native, decode_gqa_attention, mixed_gqa_attention
from oracle import inputs
from tests.conftest import assert_attn_close
from tests.golden.make_golden import INPUT_FIELDS, build_case, digest
from tests.gpu_helpers import DEV, bits, err_word, gpu_mixed_step, note, oracle_mixed

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _check(case, o, what):
    want, written = oracle_mixed(case)
    assert_attn_close(o[written], want[written], what=what)


def test_mixed_matches_golden_fixture(native_lib):
    z = np.load(os.path.join(GOLDEN, "mixed_small.npz"), allow_pickle=False)
    meta = json.loads(str(z["meta"]))
    case = build_case(meta["spec"])
    for f in INPUT_FIELDS:
        assert digest(getattr(case, f)) == meta["digests"][f], f
    note("golden mixed_small")
    kp, vp, o = gpu_mixed_step(case)
    assert digest(kp) == meta["pool_digest_k"] and digest(vp) == meta["pool_digest_v"]
    w = torch.from_numpy(z["written"])
    assert_attn_close(o[w], torch.from_numpy(z["out"])[w], what="mixed_small")


def test_mixed_config3(native_lib):
    case = inputs.config3()
    note(f"mixed config3 T={case.T}")
    kp, vp, o = gpu_mixed_step(case, max_seqlen=case.meta["max_seqlen"])
    ko, vo = case.appended_pools()
    assert torch.equal(bits(kp), bits(ko)) and torch.equal(bits(vp), bits(vo))
    _check(case, o, "config3")


@pytest.mark.parametrize("prior,new", [
    ([0], [1]), ([0], [2]), ([0], [3]), ([0], [16]), ([0], [17]), ([0], [100]),
    ([0, 0, 0], [31, 32, 33]),
    ([5, 700, 16, 2000], [1, 1, 2, 1]),              # decode-like (key-parallel) tiles
    ([100, 0, 3000, 50], [40, 1, 18, 2]),            # prefill tails of 2 and 8 rows
    ([0, 1500, 0, 64], [250, 3, 0, 129]),            # an empty sequence in the middle
], ids=lambda x: str(x))
def test_mixed_shapes(native_lib, prior, new):
    case = inputs.make_case(prior, new, seed=31)
    note(f"mixed prior={prior} new={new}")
    kp, vp, o = gpu_mixed_step(case)
    ko, vo = case.appended_pools()
    assert torch.equal(bits(kp), bits(ko)) and torch.equal(bits(vp), bits(vo))
    _check(case, o, f"mixed {prior}/{new}")


@pytest.mark.parametrize("prior,new,d", [
    ([16000, 5], [20, 1], 64),       # a prefix long enough to split over several workgroups
    ([5000, 3000], [1, 33], 128),
    ([30000], [1], 64),               # one decode row past the chunk cap (16 chunks of its keys)
    ([30000, 9, 700], [1, 1, 1], 128),
    # past 65,536 keys a wave's share of a chunk spans more than one 64-tile
    # run of lane offsets (both streams' per-run thresholds and lane tiles)
    ([70000, 70000, 3], [20, 1, 40], 64),
    ([70001, 3], [1, 17], 128),
], ids=lambda x: str(x))
def test_mixed_long_prefixes_split_keys(native_lib, prior, new, d):
    case = inputs.make_case(prior, new, seed=37, d=d)
    note(f"mixed long prefixes prior={prior} new={new} D={d}")
    kp, vp, o = gpu_mixed_step(case)
    _check(case, o, f"long {prior}/{new} D={d}")


def test_mixed_largest_batch(native_lib):
    """1,024 sequences, the kernel's limit: its plan tables (28 B per sequence)
    take LDS sized to the batch, here the largest allocation it makes."""
    g = torch.Generator().manual_seed(39)
    prior = torch.randint(0, 48, (1024,), generator=g).tolist()
    new = torch.randint(0, 3, (1024,), generator=g).tolist()
    case = inputs.make_case(prior, new, seed=39)
    note("mixed 1024 sequences")
    kp, vp, o = gpu_mixed_step(case)
    ko, vo = case.appended_pools()
    assert torch.equal(bits(kp), bits(ko)) and torch.equal(bits(vp), bits(vo))
    _check(case, o, "1024 sequences")


@pytest.mark.parametrize("B", [64, 65, 200])
def test_mixed_plan_paths_around_64_sequences(native_lib, B):
    """Batches of up to 64 sequences are planned by each wave alone (heaviest
    sequence first), larger ones by the workgroup in sequence order: prefill
    chunks with long prefixes (split keys), decode rows and empty sequences
    on both sides of the boundary."""
    g = torch.Generator().manual_seed(41 + B)
    prior = torch.randint(0, 2500, (B,), generator=g).tolist()
    new = [int(x) for x in torch.randint(0, 3, (B,), generator=g)]
    for i in range(0, B, 9):
        new[i] = 40 + 7 * (i % 5)  # prefill chunks among the decode rows
    prior[1] = 9000                   # a prefix long enough to split
    err = err_word()
    case = inputs.make_case(prior, new, seed=41 + B)
    note(f"mixed plan paths B={B} rows={sum(new)}")
    kp, vp, o = gpu_mixed_step(case, err=err)
    assert int(err.item()) == 0
    _check(case, o, f"plan paths B={B}")


@pytest.mark.parametrize("h_q,h_kv", [(14, 2), (8, 1), (8, 2)])
def test_mixed_column_groups_by_sequence(native_lib, h_q, h_kv):
    """Sequences whose longest tile has at most 32 key tiles (prior + rows <=
    512) split a tile's columns into groups of 2, longer ones into groups
    of 4: one batch on both sides of the boundary (full and partial last
    tiles, a decode row, a prefix long enough to split its keys), for 7, 8
    and 4 heads per kv head."""
    prior = [256, 257, 0, 500, 100, 511, 2000, 6000]
    new = [256, 256, 512, 13, 77, 1, 40, 20]
    err = err_word()
    case = inputs.make_case(prior, new, h_q=h_q, h_kv=h_kv, seed=43)
    note(f"mixed column groups by sequence H_q={h_q} H_kv={h_kv}")
    kp, vp, o = gpu_mixed_step(case, err=err)
    assert int(err.item()) == 0
    ko, vo = case.appended_pools()
    assert torch.equal(bits(kp), bits(ko)) and torch.equal(bits(vp), bits(vo))
    _check(case, o, f"column groups H_q={h_q} H_kv={h_kv}")


def test_mixed_batch_above_the_plan_limit_is_rejected(native_lib):
    case = inputs.make_case([2] * 1025, seed=40)
    note("mixed 1025 sequences (rejected)")
    c = case.to(DEV)
    with pytest.raises(RuntimeError, match="unsupported shape"):
        mixed_gqa_attention(c.q, c.k_pool, c.v_pool, 1, c.cu_seqlens, c.kv_lens, c.slot_ids,
                            c.block_table)


@pytest.mark.parametrize("n_pages,where", [
    (2**20 - 1, "top"),    # pools of 4 GiB - 4 KiB: one descriptor per pool, offsets near 2^32
    (2**20 + 64, "top"),   # pools past 4 GiB: the per-tile descriptor path, offsets past 2^32
], ids=["just-under-4GiB", "past-4GiB"])
def test_mixed_pools_near_and_past_4gib(native_lib, n_pages, where):
    """The kernel streams K/V through one descriptor per pool with 32-bit tile
    offsets when a pool is under 4 GiB and through per-tile descriptors
    otherwise; a case's pages placed at the top of such pools read the same
    keys as the small pool they came from."""
    case = inputs.make_case([3000, 0, 700, 40], [1, 45, 20, 3], seed=41)
    note(f"mixed pools of {n_pages} pages ({where})")
    kp_small, vp_small = case.appended_pools()
    n_small = kp_small.shape[0]
    shift = n_pages - n_small  # the case's page p lands at page p + shift
    kp = torch.empty((n_pages,) + tuple(kp_small.shape[1:]), dtype=torch.float16, device=DEV)
    vp = torch.empty_like(kp)
    kp[shift:] = kp_small.to(DEV)
    vp[shift:] = vp_small.to(DEV)
    c = case.to(DEV)
    bt = c.block_table + shift
    lib = _native.load()
    H_q, D = 14, 64
    o = torch.empty_like(c.q)
    ws = torch.empty(lib.cie_mixed_partials_bytes(case.T, H_q, D), dtype=torch.uint8, device=DEV)
    max_seqlen = int(case.new_lens.max())
    ctr = torch.zeros(lib.cie_mixed_counters(case.B, 2, max_seqlen), dtype=torch.int32, device=DEV)
    err = err_word()
    rc = lib.cie_mixed_attention(o.data_ptr(), c.q.data_ptr(), kp.data_ptr(), vp.data_ptr(),
                                 c.cu_seqlens.data_ptr(), c.kv_lens.data_ptr(), c.slot_ids.data_ptr(),
                                 bt.data_ptr(), ws.data_ptr(), ws.numel(), ctr.data_ptr(), case.B, case.T,
                                 max_seqlen, H_q, 2, D,
                                 16, n_pages, kp.stride(0), kp.stride(1), bt.stride(0),
                                 bt.shape[1], bt.shape[0], err.data_ptr(),
                                 _native.stream_handle(torch.device(DEV)))
    assert rc == 0
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    del kp, vp
    _check(case, o[0].float().cpu(), f"pools of {n_pages} pages")


def test_mixed_partials_above_2gib_in_the_low_address_word(native_lib):
    """Split tiles store partials through buffer descriptors built from the region's address.

    The partials are placed where every address's low 32-bit word has bit 31
    set; a descriptor that sign-extended that word into the high one would
    point outside the allocation.
    """
    case = inputs.make_case([3071, 6000, 0], [1, 20, 5], seed=38)
    note("mixed partials at a high low-word address")
    c = case.to(DEV)
    kp, vp = (t.to(DEV) for t in case.appended_pools())
    lib = _native.load()
    H_q, D = 14, 64
    need = lib.cie_mixed_partials_bytes(case.T, H_q, D)
    big = torch.empty(2**31 + 2 * need + 4096, dtype=torch.uint8, device=DEV)
    base = big.data_ptr()
    low = base % 2**32
    if 2**31 <= low and low + need < 2**32:
        off = 0
    else:
        off = (2**31 - low) % 2**32
    off = (off + 255) // 256 * 256
    ptr = base + off
    assert 2**31 <= ptr % 2**32 and ptr % 2**32 + need < 2**32 and off + need <= big.numel()
    o = torch.empty_like(c.q)
    ctr = torch.zeros(lib.cie_mixed_counters(case.B, 2, 20), dtype=torch.int32, device=DEV)
    rc = lib.cie_mixed_attention(o.data_ptr(), c.q.data_ptr(), kp.data_ptr(), vp.data_ptr(),
                                 c.cu_seqlens.data_ptr(), c.kv_lens.data_ptr(), c.slot_ids.data_ptr(),
                                 c.block_table.data_ptr(), ptr, need, ctr.data_ptr(), case.B, case.T,
                                 20, H_q, 2, D,
                                 16, kp.shape[0], kp.stride(0), kp.stride(1), c.block_table.stride(0),
                                 c.block_table.shape[1], c.block_table.shape[0], None,
                                 _native.stream_handle(torch.device(DEV)))
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.count_nonzero(ctr) == 0
    del big
    _check(case, o[0].float().cpu(), "partials at a high low-word address")


def test_mixed_single_rows_match_decode_kernel(native_lib):
    """L = 1 sequences through the mixed kernel equal the decode kernel on the same pool."""
    case = inputs.make_case([0, 31, 512, 3071], seed=32)
    note("mixed vs decode")
    kp, vp, om = gpu_mixed_step(case)
    c = case.to(DEV)
    od = decode_gqa_attention(c.q, kp.to(DEV), vp.to(DEV), c.attended, c.slot_ids, c.block_table)
    assert_attn_close(om, od[0].float().cpu(), atol=1e-3, rtol=1e-2, what="mixed L=1 vs decode")


@pytest.mark.parametrize("h_q,h_kv,d,ps", [(8, 8, 64, 16), (8, 1, 64, 16), (14, 2, 128, 16), (14, 2, 64, 32)])
def test_mixed_head_geometries(native_lib, h_q, h_kv, d, ps):
    case = inputs.make_case([0, 40, 300], [37, 1, 20], seed=33, h_q=h_q, h_kv=h_kv, d=d, page_size=ps)
    note(f"mixed geometry {h_q}/{h_kv} D={d} ps={ps}")
    _, _, o = gpu_mixed_step(case)
    _check(case, o, "geometry")


def test_mixed_leaves_rows_outside_sequences_untouched(native_lib):
    """Rows past cu_seqlens[-1] keep their contents (the reference never stores them)."""
    case = inputs.make_case([10, 0], [5, 3], seed=34)
    note("mixed untouched rows")
    c = case.to(DEV)
    kp, vp = case.appended_pools()
    kp, vp = kp.to(DEV), vp.to(DEV)
    T_pad = case.T + 4
    q = torch.zeros(1, T_pad, 14, 64, dtype=torch.float16, device=DEV)
    q[:, :case.T] = c.q
    o = torch.full_like(q, 7.0)
    lib = _native.load()
    ws = torch.empty(lib.cie_mixed_partials_bytes(T_pad, 14, 64), dtype=torch.uint8, device=DEV)
    ctr = torch.zeros(lib.cie_mixed_counters(case.B, 2, 16), dtype=torch.int32, device=DEV)
    rc = lib.cie_mixed_attention(o.data_ptr(), q.data_ptr(), kp.data_ptr(), vp.data_ptr(),
                                 c.cu_seqlens.data_ptr(), c.kv_lens.data_ptr(), c.slot_ids.data_ptr(),
                                 c.block_table.data_ptr(), ws.data_ptr(), ws.numel(), ctr.data_ptr(),
                                 case.B, T_pad,
                                 16, 14, 2, 64,
                                 16, kp.shape[0], kp.stride(0), kp.stride(1), c.block_table.stride(0),
                                 c.block_table.shape[1], c.block_table.shape[0], None,
                                 _native.stream_handle(torch.device(DEV)))
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.all(o[0, case.T:] == 7.0)
    _check(case, o[0, :case.T].float().cpu(), "untouched")


def test_mixed_rows_beyond_max_seqlen_are_flagged(native_lib):
    case = inputs.make_case([0], [40], seed=35)
    note("mixed max_seqlen flag")
    err = err_word()
    gpu_mixed_step(case, max_seqlen=16, err=err)
    assert int(err.item()) & 2


def test_mixed_counters_return_to_zero(native_lib):
    """Multi-chunk tiles (long prefixes) leave their arrival counters zero."""
    case = inputs.make_case([6000, 0, 2500, 700, 30000], [40, 1, 1, 18, 1], seed=36)
    note("mixed counters")
    c = case.to(DEV)
    kp, vp = (t.to(DEV) for t in case.appended_pools())
    from custom_inference_engine_amd import mixed_gqa_attention
    ctr = torch.zeros(_native.load().cie_mixed_counters(case.B, 2, 40), dtype=torch.int32, device=DEV)
    for _ in range(2):
        o = mixed_gqa_attention(c.q, kp, vp, 40, c.cu_seqlens, c.kv_lens, c.slot_ids, c.block_table,
                                counters=ctr)
        torch.cuda.synchronize()
        assert torch.count_nonzero(ctr) == 0
    _check(case, o[0].float().cpu(), "mixed counters")


def test_mixed_stale_counters_are_flagged_and_cleared(native_lib):
    """Arrival words preloaded far above any chunk count raise CIE_ERRBIT_SPLIT in a
    call with multi-chunk tiles; every chunk of those tiles sees its word stale, so the
    call clears the words it uses and the next call is correct with no error bit."""
    case = inputs.make_case([6000, 0, 2500, 700, 30000], [40, 1, 1, 18, 1], seed=37)
    note("mixed stale counters")
    c = case.to(DEV)
    kp, vp = (t.to(DEV) for t in case.appended_pools())
    from custom_inference_engine_amd import mixed_gqa_attention
    n = _native.load().cie_mixed_counters(case.B, 2, 40)
    ctr = torch.zeros(n, dtype=torch.int32, device=DEV)
    ctr[: n // 2] = 1000  # every arrival word
    err = err_word()
    mixed_gqa_attention(c.q, kp, vp, 40, c.cu_seqlens, c.kv_lens, c.slot_ids, c.block_table,
                        counters=ctr, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 8, "CIE_ERRBIT_SPLIT expected"
    assert torch.count_nonzero(ctr[n // 2:]) == 0  # stale words back to zero
    used = ctr[: n // 2] == 0
    assert bool(used.any())
    err.zero_()
    o = mixed_gqa_attention(c.q, kp, vp, 40, c.cu_seqlens, c.kv_lens, c.slot_ids, c.block_table,
                            counters=ctr, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    _check(case, o[0].float().cpu(), "call after the stale one")


def test_mixed_counters_preloaded_negative_are_flagged_then_reset(native_lib):
    """Arrival words at -1 are flagged by the call that finds them; after the caller
    re-zeroes the buffer the next call is correct with no error bit."""
    case = inputs.make_case([6000, 0, 2500, 700, 30000], [40, 1, 1, 18, 1], seed=38)
    note("mixed counters preloaded -1")
    c = case.to(DEV)
    kp, vp = (t.to(DEV) for t in case.appended_pools())
    from custom_inference_engine_amd import mixed_gqa_attention
    n = _native.load().cie_mixed_counters(case.B, 2, 40)
    ctr = torch.zeros(n, dtype=torch.int32, device=DEV)
    ctr[: n // 2] = -1  # every arrival word
    err = err_word()
    mixed_gqa_attention(c.q, kp, vp, 40, c.cu_seqlens, c.kv_lens, c.slot_ids, c.block_table,
                        counters=ctr, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) & 8, "CIE_ERRBIT_SPLIT expected"
    ctr.zero_()
    err.zero_()
    o = mixed_gqa_attention(c.q, kp, vp, 40, c.cu_seqlens, c.kv_lens, c.slot_ids, c.block_table,
                            counters=ctr, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    assert torch.count_nonzero(ctr) == 0
    _check(case, o[0].float().cpu(), "call after the reset")


def _split_partial_rows(prior, new, h_q, h_kv, n_qtiles):
    """Partial rows each sequence's split tiles take, tile by tile: a tile of
    `rows` rows with k >= 2 chunks holds rows * H_q * k; k = clamp(ceil(pairs
    / per), 1, 16) for the tile's 32-key steps, per = 4 waves x 12 steps (one
    column tile: CIE_MIXED_NARROW_PAIRS) or 4 x 24 (wider)."""
    G = h_q // h_kv
    out = []
    for c, L in zip(prior, new):
        r = 0
        for t in range(min((L + 15) // 16, n_qtiles)):
            rows = min(16, L - 16 * t)
            n_ctiles = (rows * G + 15) // 16
            pairs = ((c + 16 * t + rows + 15) // 16 + 1) // 2
            per = 4 * 12 if n_ctiles == 1 else 4 * 24
            k = max(1, min(16, -(-pairs // per)))
            if k > 1:
                r += rows * h_q * k
        out.append(r)
    return out


def _budget_bytes(rows, d):
    """Bytes of a partials buffer that holds exactly `rows` rows (three 256-byte aligned regions)."""
    return 3 * 256 + rows * 4 * (d + 2)


def _mixed_with_budget(case, nbytes, max_seqlen, h_q=14, h_kv=2, d=64):
    """One mixed call through the C ABI with a partials budget of `nbytes`,
    inside a buffer with 4 KiB of 0xFF canary past it; returns (o, the
    buffer's first nbytes, canary intact, counters clean)."""
    c = case.to(DEV)
    kp, vp = (t.to(DEV) for t in case.appended_pools())
    lib = _native.load()
    buf = torch.full((nbytes + 4096,), 0xFF, dtype=torch.uint8, device=DEV)
    o = torch.empty_like(c.q)
    ctr = torch.zeros(lib.cie_mixed_counters(case.B, h_kv, max_seqlen), dtype=torch.int32, device=DEV)
    err = err_word()
    rc = lib.cie_mixed_attention(o.data_ptr(), c.q.data_ptr(), kp.data_ptr(), vp.data_ptr(),
                                 c.cu_seqlens.data_ptr(), c.kv_lens.data_ptr(), c.slot_ids.data_ptr(),
                                 c.block_table.data_ptr(), buf.data_ptr() if nbytes else None, nbytes,
                                 ctr.data_ptr(), case.B, case.T, max_seqlen, h_q, h_kv, d,
                                 16, kp.shape[0], kp.stride(0), kp.stride(1), c.block_table.stride(0),
                                 c.block_table.shape[1], c.block_table.shape[0], err.data_ptr(),
                                 _native.stream_handle(torch.device(DEV)))
    assert rc == 0
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    canary = bool(torch.all(buf[nbytes:] == 0xFF))
    return o[0].float().cpu(), buf[:nbytes].cpu(), canary, int(torch.count_nonzero(ctr)) == 0


def _written_m_rows(ws, cap):
    """Rows of part_m (the buffer's first region) a call wrote: 0xFF bytes are NaN, written m never is."""
    m = ws[:4 * cap].view(torch.float32)
    return (~torch.isnan(m)).nonzero().flatten()


def test_mixed_partials_decode_rows_default_budget(native_lib):
    """A batch of mostly long decode rows (12 rows of 6,000-8,200 keys, 7 to
    11 chunks each, and one 8-token prefill): the default budget's floor of
    16 rows per token for the first 64 tokens lets every decode row split —
    the call writes exactly the rows all their chunks need — and the result
    matches the oracle."""
    prior = [0] + [6000 + 200 * i for i in range(12)]
    new = [8] + [1] * 12
    case = inputs.make_case(prior, new, seed=45)
    ms = 8
    need = _split_partial_rows(prior, new, 14, 2, 1)
    assert all(r > 0 for r in need[1:]) and need[0] == 0
    nbytes = _native.load().cie_mixed_partials_bytes(case.T, 14, 64)
    assert 2 * case.T * 14 < sum(need) <= (nbytes - 768) // (4 * 66)
    note(f"mixed decode rows, default partials budget ({nbytes} bytes, {sum(need)} rows)")
    o, ws, canary, clean = _mixed_with_budget(case, nbytes, ms)
    assert canary and clean
    rows = _written_m_rows(ws, (nbytes - 768) // (4 * 66))
    assert rows.numel() == sum(need) and int(rows.max()) == sum(need) - 1
    _check(case, o, "decode rows, default partials budget")


def test_mixed_partials_config3_default_budget(native_lib):
    """Config 3 takes 504 partial rows (its decode rows split, its prefill
    chunks do not), well inside the default budget (at 1,052 tokens: 2 rows
    per token and head, under 8 MB): the call writes exactly rows [0, 504)
    of part_m, nothing past its buffer, and matches the oracle."""
    case = inputs.config3()
    ms = case.meta["max_seqlen"]
    need = _split_partial_rows(case.kv_lens.tolist(), case.new_lens.tolist(), 14, 2, (ms + 15) // 16)
    assert sum(need) == 504
    nbytes = _native.load().cie_mixed_partials_bytes(case.T, 14, 64)
    assert nbytes <= 8_000_000
    note(f"mixed config3 default partials budget ({nbytes} bytes)")
    o, ws, canary, clean = _mixed_with_budget(case, nbytes, ms)
    assert canary and clean
    cap = (nbytes - 768) // (4 * 66)
    rows = _written_m_rows(ws, cap)
    assert rows.numel() == 504 and int(rows.max()) == 503
    _check(case, o, "config3, default partials budget")


@pytest.mark.parametrize("B", [24, 90])
def test_mixed_partials_budget_splits_a_prefix_of_the_batch(native_lib, B):
    """Sequences take their partial rows in sequence order; one whose rows
    would end past the budget, and every split sequence after it, runs
    unsplit.  Budgets of 0, one row short of the need, a part of it and
    exactly the need give the oracle's output, write exactly the fitting
    prefix's rows and nothing past the buffer — for the wave plan (B <= 64)
    and the block plan."""
    g = torch.Generator().manual_seed(47 + B)
    prior = torch.randint(0, 3000, (B,), generator=g).tolist()
    new = [int(x) for x in torch.randint(1, 3, (B,), generator=g)]
    prior[2], new[2] = 9000, 20      # a prefill tail whose tiles split
    prior[5], new[5] = 30000, 1      # a decode row of 16 chunks (the cap)
    new[7] = 0                       # an empty sequence
    case = inputs.make_case(prior, new, seed=47 + B)
    ms = int(max(new))
    P = _split_partial_rows(prior, new, 14, 2, (ms + 15) // 16)
    need = sum(P)
    assert need > 0 and P[2] > 0 and P[5] == 14 * 16
    want, written = oracle_mixed(case)
    for cap in (0, need - 1, need // 3, need):
        nbytes = 0 if cap == 0 else _budget_bytes(cap, 64)
        note(f"mixed B={B} partials budget {cap} of {need} rows")
        o, ws, canary, clean = _mixed_with_budget(case, nbytes, ms)
        assert canary and clean, cap
        fit, pre = 0, 0
        for p in P:  # the plan's rule: prefix over all earlier sequences
            if p and pre + p <= cap:
                fit += p
            pre += min(p, cap + 1)
        if cap:
            rows = _written_m_rows(ws, cap)
            assert rows.numel() == fit, (cap, rows.numel(), fit)
            assert fit == 0 or int(rows.max()) == fit - 1
        assert_attn_close(o[written], want[written], what=f"budget {cap} of {need}")


def test_mixed_partials_budget_through_the_python_api(native_lib):
    """`mixed_gqa_attention(..., partials_bytes=)`: no budget (nothing splits),
    a tight one and the default give the oracle's output; a negative budget is
    refused on the host."""
    case = inputs.make_case([9000, 700, 3000, 20000], [20, 1, 2, 1], seed=71)
    c = case.to(DEV)
    kp, vp = (t.to(DEV) for t in case.appended_pools())
    want, written = oracle_mixed(case)
    for nbytes in (0, _budget_bytes(14 * 16, 64), None):
        note(f"mixed python api partials_bytes={nbytes}")
        o = mixed_gqa_attention(c.q, kp, vp, 20, c.cu_seqlens, c.kv_lens, c.slot_ids, c.block_table,
                                partials_bytes=nbytes)
        torch.cuda.synchronize()
        assert_attn_close(o[0].float().cpu()[written], want[written], what=f"partials_bytes={nbytes}")
    with pytest.raises(AssertionError):
        mixed_gqa_attention(c.q, kp, vp, 20, c.cu_seqlens, c.kv_lens, c.slot_ids, c.block_table,
                            partials_bytes=-1)
