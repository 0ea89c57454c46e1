"""The C-ABI library: it loads, exports every declared symbol, and its host-side
validation rejects bad arguments before launching anything (no GPU needed)."""
import ctypes
import os
import re

import pytest

from custom_inference_engine_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cie_paged_attention.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cie_\w+)\s*\(", text)))


def test_header_declares_the_hot_path():
    names = declared_functions()
    for want in ("cie_kv_append_decode", "cie_kv_append_tokens", "cie_paged_decode",
                 "cie_paged_decode_append", "cie_paged_decode_max_splits",
                 "cie_paged_decode_partials_bytes", "cie_mixed_attention",
                 "cie_paged_decode_qkv_rope", "cie_kv_append_tokens_qkv_rope",
                 "cie_mixed_partials_bytes", "cie_mixed_counters", "cie_abi_version",
                 "cie_status_string"):
        assert want in names


def test_library_exports_every_declared_symbol(native_lib):
    missing = [n for n in declared_functions() if not hasattr(native_lib, n)]
    assert not missing, missing
    # and the ctypes table covers the same set, so every entry point is typed
    assert set(_native._SIGNATURES) == set(declared_functions())
    # bench.py's measurement kernels live in a library of their own
    for name in ("cie_bench_gather_read", "cie_probe_gather_read", "cie_bench_step_probe"):
        assert not hasattr(native_lib, name), name


def test_single_hip_runtime_in_process(native_lib):
    """The library binds to torch's HIP runtime (one libamdhip64 mapping)."""
    maps = open("/proc/self/maps").read()
    paths = {line.split()[-1] for line in maps.splitlines() if "libamdhip64" in line}
    assert len(paths) == 1, paths


def test_version_and_status_strings(native_lib):
    assert native_lib.cie_abi_version() == _native.ABI_VERSION
    assert native_lib.cie_status_string(0) == b"ok"
    assert b"invalid" in native_lib.cie_status_string(-1)
    assert b"unsupported" in native_lib.cie_status_string(-2)


def test_workspace_sizes(native_lib):
    # (B, H_q, S, D + 2) fp32 partial state, 256-byte aligned regions
    n = native_lib.cie_paged_decode_partials_bytes(32, 14, 64, 16)
    assert n >= 32 * 14 * 16 * 66 * 4 and n % 256 == 0
    assert native_lib.cie_paged_decode_partials_bytes(-1, 14, 64, 16) == -1
    assert native_lib.cie_paged_decode_max_splits() >= 16
    # mixed: a budget of 2 chunk rows (D + 2 floats) per token and q head —
    # 7.8 MB at config 3's 1,052 tokens — capped at 2,097,088 rows
    n = native_lib.cie_mixed_partials_bytes(1052, 14, 64)
    assert 2 * 1052 * 14 * 66 * 4 <= n <= 8_000_000 and n % 256 == 0
    assert native_lib.cie_mixed_partials_bytes(10**6, 64, 128) < 2_097_088 * 130 * 4 + 1024
    assert native_lib.cie_mixed_partials_bytes(0, 14, 64) >= 0
    assert native_lib.cie_mixed_partials_bytes(10, 0, 64) == -1
    # small batches (mostly decode rows): 16 rows (a row's most chunks) for
    # each of the first 64 tokens, so every decode row can split
    row = 66 * 4
    assert native_lib.cie_mixed_partials_bytes(28, 14, 64) >= 16 * 28 * 14 * row
    assert native_lib.cie_mixed_partials_bytes(100, 14, 64) >= 16 * 64 * 14 * row
    assert native_lib.cie_mixed_partials_bytes(100, 14, 64) < 16 * 64 * 14 * row + 1024
    # an arrival word and a stale word per (tile, column group)
    n = native_lib.cie_mixed_counters(32, 2, 256)
    assert n >= 2 * 32 * 2 * 16 and n % 2 == 0


def _decode_args(**over):
    a = dict(o=144, q=16, k=32, v=48, lens=64, slots=80, bt=96, ws=112, ctr=128, B=1, H_q=14, H_kv=2, D=64,
             page_size=16, n_pages=64, page_stride=2048, head_stride=1024, bt_stride=64,
             bt_width=64, n_slots=2, n_splits=4)
    a.update(over)
    return a


def _call_decode(lib, a):
    # fake, never-dereferenced device addresses: these calls must fail validation on the host
    return lib.cie_paged_decode(a["o"], a["q"], a["k"], a["v"], a["lens"], a["slots"], a["bt"],
                                a["ws"], a["ctr"], a["B"], a["H_q"], a["H_kv"], a["D"], a["page_size"],
                                a["n_pages"], a["page_stride"], a["head_stride"], a["bt_stride"],
                                a["bt_width"], a["n_slots"], a["n_splits"], None, None)


@pytest.mark.parametrize("over,code", [
    ({"H_q": 13}, -1),                 # H_q not a multiple of H_kv
    ({"n_splits": 0}, -1),
    ({"bt_stride": 8}, -1),            # stride below width
    ({"page_size": 8}, -2),            # pages must hold whole 16-key tiles
    ({"D": 96}, -2),                   # head_dim outside the built set
    ({"H_q": 34, "H_kv": 2}, -2),      # more than 16 query heads per kv head
    ({"q": 18}, -1),                   # q not 16-byte aligned
    ({"o": 8}, -1),                    # o not 16-byte aligned
    ({"lens": 0}, -1),                 # null index pointer
    ({"ctr": 0}, -1),                  # split counters needed when n_splits > 1
    ({"n_splits": 65}, -2),            # above the merge's split limit
])
def test_decode_rejects_bad_arguments_without_launching(native_lib, over, code):
    assert _call_decode(native_lib, _decode_args(**over)) == code


def test_decode_empty_batch_is_a_noop(native_lib):
    assert _call_decode(native_lib, _decode_args(B=0)) == 0


def test_fused_decode_rejects_missing_new_rows(native_lib):
    a = _decode_args()
    rc = native_lib.cie_paged_decode_append(a["o"], a["q"], a["k"], a["v"], None, None, 128, 64, 128, 64,
                                            a["lens"], a["slots"], a["bt"], a["ws"], a["ctr"], 1, 14, 2, 64, 16,
                                            64, 2048, 1024, 64, 64, 2, 4, None, None)
    assert rc == -1
    rc = native_lib.cie_paged_decode_append(a["o"], a["q"], a["k"], a["v"], 16, 24, 128, 64, 128, 64,
                                            a["lens"], a["slots"], a["bt"], a["ws"], a["ctr"], 1, 14, 2, 64, 16,
                                            64, 2048, 1024, 64, 64, 2, 4, None, None)
    assert rc == -1  # v_new not 16-byte aligned


def test_append_and_mixed_reject_bad_arguments(native_lib):
    lib = native_lib
    # negative row count
    assert lib.cie_kv_append_tokens(8, 8, 8, 8, 64, 64, 64, 64, 8, 8, -1, 2, 16, 64, 10, 2048,
                                    1024, None, None) == -1
    # zero rows: nothing to do
    assert lib.cie_kv_append_tokens(8, 8, 8, 8, 64, 64, 64, 64, 8, 8, 0, 2, 16, 64, 10, 2048,
                                    1024, None, None) == 0
    assert lib.cie_kv_append_decode(8, 8, 8, 8, 64, 64, 64, 64, 8, 8, 8, 1, 2, 16, 64, 10, 2048,
                                    1024, 4, 8, 2, None, None) == -1  # bt_stride < bt_width
    # mixed: G = 14 > 8 is outside the built set
    assert lib.cie_mixed_attention(16, 16, 16, 16, 8, 8, 8, 8, 16, 4096, 32, 1, 4, 4, 14, 1, 64, 16, 10,
                                   1024, 1024, 10, 10, 2, None, None) == -2
    # mixed: counters are required
    assert lib.cie_mixed_attention(16, 16, 16, 16, 8, 8, 8, 8, 16, 4096, None, 1, 4, 4, 14, 2, 64, 16, 10,
                                   1024, 1024, 10, 10, 2, None, None) == -1
    # mixed: a partials budget without a buffer, and a negative budget
    assert lib.cie_mixed_attention(16, 16, 16, 16, 8, 8, 8, 8, None, 4096, 32, 1, 4, 4, 14, 2, 64, 16, 10,
                                   1024, 1024, 10, 10, 2, None, None) == -1
    assert lib.cie_mixed_attention(16, 16, 16, 16, 8, 8, 8, 8, 16, -1, 32, 1, 4, 4, 14, 2, 64, 16, 10,
                                   1024, 1024, 10, 10, 2, None, None) == -1


def _call_decode_rope(lib, qkv_stride=1152, cos=32, cs_stride=64, B=1, D=64):
    # fake, never-dereferenced device addresses: must fail validation on the host
    return lib.cie_paged_decode_qkv_rope(144, 16, qkv_stride, cos, 48, cs_stride, 64, 80, 96, 112, 128,
                                         160, 176, B, 14, 2, D, 16, 64, 2048, 1024, 64, 64, 2, 4,
                                         None, None)


def _call_tokens_rope(lib, qkv=16, T=3, D=64, qkv_stride=1152):
    return lib.cie_kv_append_tokens_qkv_rope(144, 64, 80, qkv, qkv_stride, 32, 48, 64, 96, 112, T, 14, 2,
                                             16, D, 64, 2048, 1024, None, None)


def test_rope_entry_points_reject_bad_arguments_without_launching(native_lib):
    lib = native_lib
    assert _call_decode_rope(lib, qkv_stride=64) == -1      # row stride below q|k|v width
    assert _call_decode_rope(lib, qkv_stride=1156) == -1    # row stride not a multiple of 8
    assert _call_decode_rope(lib, cos=40) == -1             # cos not 16-byte aligned
    assert _call_decode_rope(lib, cs_stride=32) == -1       # cos row shorter than D
    assert _call_decode_rope(lib, B=0) == 0                 # empty batch: no-op
    assert _call_tokens_rope(lib, D=72, qkv_stride=1296) == -2  # D not a multiple of 16
    assert _call_tokens_rope(lib, qkv=24) == -1             # qkv not 16-byte aligned
    assert _call_tokens_rope(lib, T=0) == 0                 # no tokens: no-op
    assert _call_tokens_rope(lib, T=-1) == -1


CIE_EUNSUPPORTED, CIE_ESCRATCH = -2, -3
SCRATCH_PARTIALS, SCRATCH_WORDS = 4 << 20, 16384


def _call_noalloc(lib, B, H_q, H_kv, n_splits):
    # fake, never-dereferenced device addresses: a refused size returns before any device call
    return lib.cie_paged_decode_append_noalloc(16, 16, 16, 16, 16, 16, 64, 64, 64, 64, 16, 16, 16, B, H_q,
                                               H_kv, 64, 16, 64, 2048, 1024, 64, 64, 65, n_splits, None, None)


@pytest.mark.parametrize("n_splits", [1, 4, 16])
@pytest.mark.parametrize("h_q,h_kv", [(14, 1), (14, 2), (32, 8)])
def test_noalloc_limit_is_exact(native_lib, n_splits, h_q, h_kv):
    """cie_paged_decode_noalloc_limit gives the largest batch the allocation-free entry
    point accepts: `limit` gets past every size check (here, with no GPU, it then fails at
    the device), `limit + 1` is refused on the host."""
    lib = native_lib
    limit = lib.cie_paged_decode_noalloc_limit(h_q, h_kv, 64, n_splits)
    assert 0 < limit <= 65535
    if n_splits == 1:  # no partials, no counters: only the kernel's grid bound
        assert limit == 65535
    else:
        assert lib.cie_paged_decode_partials_bytes(limit, h_q, 64, n_splits) <= SCRATCH_PARTIALS
        assert 2 * limit * h_kv <= SCRATCH_WORDS
        assert (lib.cie_paged_decode_partials_bytes(limit + 1, h_q, 64, n_splits) > SCRATCH_PARTIALS
                or 2 * (limit + 1) * h_kv > SCRATCH_WORDS)
    assert _call_noalloc(lib, limit + 1, h_q, h_kv, n_splits) in (CIE_ESCRATCH, CIE_EUNSUPPORTED)
    assert _call_noalloc(lib, limit, h_q, h_kv, n_splits) not in (CIE_ESCRATCH, CIE_EUNSUPPORTED, -1)


def test_noalloc_limit_rejects_impossible_arguments(native_lib):
    lib = native_lib
    assert lib.cie_paged_decode_noalloc_limit(14, 2, 64, lib.cie_paged_decode_max_splits() + 1) == -1
    assert lib.cie_paged_decode_noalloc_limit(14, 3, 64, 4) == -1  # H_q not a multiple of H_kv
    assert lib.cie_paged_decode_noalloc_limit(14, 2, 64, 0) == -1


def test_plan_rejects_what_it_cannot_hold(native_lib):
    """cie_paged_decode_plan checks its sizes on the host (fake addresses, never read)."""
    lib = native_lib
    # more sequences than one plan holds
    assert lib.cie_paged_decode_plan(16, 16, 16, 16, 1025, 2, 16, 64, 64, 64, 2000, 1,
                                     lib.cie_paged_decode_plan_workgroups(1025, 2, 1), None, None) == -2
    # fewer workgroups than (sequence, kv head) groups; a grid not a multiple of H_kv
    assert lib.cie_paged_decode_plan(16, 16, 16, 16, 4, 2, 16, 64, 64, 64, 10, 1, 6, None, None) == -1
    assert lib.cie_paged_decode_plan(16, 16, 16, 16, 4, 2, 16, 64, 64, 64, 10, 1, 9, None, None) == -1
    assert lib.cie_paged_decode_plan(16, 16, 16, 16, 0, 2, 16, 64, 64, 64, 10, 1, 8, None, None) == 0
    # the planned launch wants a plan and a grid of at least one workgroup per group
    assert lib.cie_paged_decode_planned(16, 16, 16, 16, None, 16, 16, 16, 4, 14, 2, 64, 16, 64, 2048,
                                        1024, 64, 64, 8, None, None) == -1
    assert lib.cie_paged_decode_planned(16, 16, 16, 16, 16, 16, 16, 16, 4, 14, 2, 64, 16, 64, 2048,
                                        1024, 64, 64, 6, None, None) == -1
    assert lib.cie_paged_decode_plan_workgroups(4, 2, 65) == -1
    assert lib.cie_paged_decode_plan_workgroups(4, 2, 16) == 128
    assert lib.cie_paged_decode_plan_bytes(256) == 256 * (8 + 4 * 64) * 4


def test_mixed_plan_rejects_bad_arguments_without_launching(native_lib):
    """cie_mixed_plan / cie_mixed_attention_planned check sizes and pointers on
    the host (fake addresses, never read)."""
    lib = native_lib
    need = lib.cie_mixed_plan_bytes(4, 100)
    # header + 8 words per item, room for every item of 100 tokens in 4 sequences:
    # (ceil(100/16) + 4) tiles x 8 column groups x 16 chunks
    assert need == (8 + 8 * (7 + 4) * 8 * 16) * 4
    assert lib.cie_mixed_plan_bytes(0, 0) == 32
    assert lib.cie_mixed_plan_bytes(-1, 100) == -1 and lib.cie_mixed_plan_bytes(1025, 100) == -1

    def plan(**over):
        a = dict(plan=4096, plan_bytes=need, cu=16, kvl=32, slots=48, B=4, T=100, ms=40, H_q=14, H_kv=2, D=64,
                 ps=16, bt_width=64, n_slots=8, pbytes=0)
        a.update(over)
        return lib.cie_mixed_plan(a["plan"], a["plan_bytes"], a["cu"], a["kvl"], a["slots"], a["B"], a["T"],
                                  a["ms"], a["H_q"], a["H_kv"], a["D"], a["ps"], a["bt_width"], a["n_slots"],
                                  a["pbytes"], None, None)
    assert plan(plan_bytes=need - 4) == -1      # too small for the batch's items
    assert plan(plan=None) == -1
    assert plan(plan=4104) == -1                # not 16-byte aligned
    assert plan(pbytes=-1) == -1
    assert plan(B=1025, plan_bytes=1 << 30) == -2  # more sequences than a launch plans
    assert plan(H_q=14, H_kv=1) == -2           # G = 14 is outside the built set
    assert plan(B=0) == 0 and plan(T=0) == 0    # empty batch: nothing to plan

    def planned(**over):
        a = dict(plan=4096, plan_bytes=need, counters=8192)
        a.update(over)
        return lib.cie_mixed_attention_planned(16, 16, 16, 16, a["plan"], a["plan_bytes"], 8, None, 0,
                                               a["counters"], 4, 100, 40, 14, 2, 64, 16, 64, 1024, 1024,
                                               64, 64, 8, None, None)
    assert planned(plan=None) == -1
    assert planned(plan_bytes=need - 4) == -1
    assert planned(counters=None) == -1
