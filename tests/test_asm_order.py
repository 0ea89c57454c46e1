"""The split merge's ordering, checked in this build's own gfx950 assembly (CPU).

The decode and mixed kernels publish a split's partial state with agent-scope
(sc1) stores and then count the split in with a relaxed agent-scope
``fetch_add`` (``arrive_last`` in csrc/cie_common.h).  Nothing in the HIP
memory model orders relaxed stores before a relaxed RMW, so the kernels rely
on the hardware order: every store has completed (``s_waitcnt vmcnt(0)``)
before the atomic is issued, and the merging workgroup reads the partials
only with sc1 loads issued after the atomic returned.  This test compiles the
kernel sources to gfx950 assembly with the library's own flags and checks, in
every kernel that elects a last arriver, that

  * the arrival atomic (the first returning ``global_atomic_add``) has a
    ``s_waitcnt`` with ``vmcnt(0)`` after the last vector-memory store before it;
  * every store of the partial state carries sc1, and no L2 writeback or
    invalidate (``buffer_wbl2`` / ``buffer_inv``) is emitted;
  * the merge's partial loads (sc1 loads after the atomic) come after a
    ``vmcnt(0)`` wait on the atomic's result.
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

from custom_inference_engine_amd import _build

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")

STORE = re.compile(r"^\s*(global|buffer|flat)_store\w*")
ATOMIC_RET = re.compile(r"^\s*global_atomic_add\b.*\bsc0\b")
WAIT_VM0 = re.compile(r"^\s*s_waitcnt\b.*\bvmcnt\(0\)")
SC1_LOAD = re.compile(r"^\s*(global|buffer)_load\w*.*\bsc1\b")


def _assembly(src: str, tmp_path) -> str:
    out = tmp_path / (os.path.basename(src) + ".s")
    flags = [f for f in _build.HIPCC_FLAGS if f != "-fPIC"]
    cmd = [HIPCC, *flags, "-I", _build.INCLUDE, "-I", _build.CSRC, "--offload-device-only", "-S",
           os.path.join(_build.CSRC, src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-4000:]
    return out.read_text()


def _kernels(asm: str) -> dict[str, list[str]]:
    """Kernel symbol -> its instruction lines (label to .Lfunc_end)."""
    out, name, body = {}, None, []
    for line in asm.splitlines():
        m = re.match(r"^(_Z\w+):", line)
        if m:
            name, body = m.group(1), []
            continue
        if name is not None:
            if line.startswith(".Lfunc_end"):
                out[name] = body
                name = None
            else:
                body.append(line)
    return out


def _check_arrival(name: str, body: list[str]) -> None:
    """Every arrival atomic — a returning atomic add whose winner path reads
    partials with sc1 loads before the next returning atomic — waits for the
    stores issued since the previous atomic (vmcnt(0) after the last of them),
    and the partial loads after it wait for its value.  Returning atomics with
    no sc1 loads after them (a work queue's fetch) publish nothing and are not
    held to this."""
    atoms = [i for i, l in enumerate(body) if ATOMIC_RET.match(l)]
    assert atoms, f"{name}: no returning atomic"
    arrivals = []
    for k, a in enumerate(atoms):
        end = atoms[k + 1] if k + 1 < len(atoms) else len(body)
        if any(SC1_LOAD.match(l) for l in body[a + 1:end]):
            arrivals.append((k, a))
    assert arrivals, f"{name}: no arrival atomic"
    stores_checked = 0
    for k, a in arrivals:
        # the last store before the arrival must be complete before the first
        # returning atomic after it (the arrival, or a stale-path atomic laid
        # out ahead of it)
        last = max((i for i in range(a) if STORE.match(body[i])), default=None)
        if last is not None:
            first_atom = min(i for i in atoms if i > last)
            assert any(WAIT_VM0.match(l) for l in body[last + 1:first_atom]), \
                f"{name}: a store before the arrival atomic is not waited for: {body[last].strip()}"
            stores_checked += 1
        later = body[a + 1:]
        first_load = next(i for i, l in enumerate(later) if SC1_LOAD.match(l))
        assert any(WAIT_VM0.match(l) for l in later[:first_load]), \
            f"{name}: partial loads issued before the arrival atomic returned"
    assert stores_checked, f"{name}: no partial store before an arrival atomic"


@pytest.mark.parametrize("src,kernel", [("paged_decode.hip", "decode_kernel"),
                                         ("mixed_attention.hip", "mixed_attention_kernel")])
def test_partials_complete_before_arrival(src, kernel, tmp_path):
    asm = _assembly(src, tmp_path)
    assert "buffer_wbl2" not in asm and "buffer_inv" not in asm
    kernels = {n: b for n, b in _kernels(asm).items() if kernel in n}
    assert kernels, f"no {kernel} in the assembly"
    for name, body in kernels.items():
        _check_arrival(name, body)
        # partial stores are agent-scope: every store of the merge path carries sc1,
        # except the output o (plain global stores of fp16) and the pool append
        partial_stores = [l for l in body if STORE.match(l) and "dwordx4" in l and "buffer_store" in l]
        assert partial_stores and all("sc1" in l for l in partial_stores), name


FMA_MIX_F16 = re.compile(r"^\s*v_(fma|mad)_mix(lo|hi)_f16\b")


@pytest.mark.parametrize("src,kernel", [("paged_decode.hip", "decode_kernel"),
                                         ("kv_append.hip", "rope")])
def test_rope_rounds_through_fp32(src, kernel, tmp_path):
    """RoPE outputs are x*cos + rotate_half(x)*sin rounded to fp32 and then to fp16,
    as the reference's fp32 apply_rotary_pos_emb followed by the fp16 cast.  A fused
    v_fma_mixlo_f16 / v_fma_mixhi_f16 rounds the exact sum straight to fp16 and
    differs from that in the last bit now and then, so none may appear in a kernel
    that rotates (the compiler formed them from the FMA and the conversion until
    rope8 made the fp32 value opaque)."""
    asm = _assembly(src, tmp_path)
    kernels = {n: b for n, b in _kernels(asm).items() if kernel in n}
    assert kernels, f"no {kernel} kernel in {src}"
    for name, body in kernels.items():
        fused = [l.strip() for l in body if FMA_MIX_F16.match(l)]
        assert not fused, f"{name}: {len(fused)} single-rounding fp16 FMAs, e.g. {fused[0]}"


PRELOAD = re.compile(r"^\s*\.amdhsa_user_sgpr_kernarg_preload_length\s+(\d+)")


def test_decode_start_arguments_are_preloaded(tmp_path):
    """decode_kernel takes the pointers its first load is indexed by (slot ids,
    plan) and the plan's grid size as three scalar arguments ahead of its
    parameter struct, and the library is built to preload three kernel
    arguments into SGPRs: every decode kernel's descriptor must preload their
    5 dwords, or the start's first load waits on a kernel-argument load again."""
    asm = _assembly("paged_decode.hip", tmp_path)
    lengths, name = {}, None
    for line in asm.splitlines():
        m = re.match(r"^\s*\.amdhsa_kernel\s+(\S+)", line)
        if m:
            name = m.group(1)
        m = PRELOAD.match(line)
        if m and name is not None:
            lengths[name] = int(m.group(1))
    decode = {n: v for n, v in lengths.items() if "decode_kernel" in n}
    assert decode, "no decode_kernel descriptor in the assembly"
    assert all(v == 5 for v in decode.values()), decode
