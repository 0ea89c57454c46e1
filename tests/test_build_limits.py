"""Build-time limits of the kernels (CPU: hipcc only, nothing runs).

The mixed kernel plans a batch in LDS (plan tables of up to kMaxSeqs
sequences beside its static arrays).  A build whose LDS could exceed what one
gfx950 workgroup may have (160 KiB) must not compile: an 8-wave build of the
mixed kernel once asked for 170,004 bytes at 1,024 sequences and its dispatch
was rejected on the GPU.  The shipped build's static LDS must match the
kernel's own account of it (MixedLds), so the bound covers what the compiler
allocates.
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
SRC = os.path.join(_build.CSRC, "mixed_attention.hip")


def _compile(tmp_path, *defines):
    flags = [f for f in _build.HIPCC_FLAGS if f != "-fPIC"]
    cmd = [HIPCC, *flags, *(f"-D{d}" for d in defines), "-I", _build.INCLUDE, "-I", _build.CSRC,
           "--offload-device-only", "-c", SRC, "-o", str(tmp_path / "mixed.o"),
           "-Rpass-analysis=kernel-resource-usage"]
    return subprocess.run(cmd, capture_output=True, text=True)


def test_mixed_build_past_the_lds_budget_does_not_compile(tmp_path):
    res = _compile(tmp_path, "CIE_MIXED_WAVES=8")
    assert res.returncode != 0
    assert "exceed a workgroup's LDS" in res.stderr


def test_shipped_mixed_build_plans_its_largest_batch_within_lds(tmp_path):
    res = _compile(tmp_path)
    assert res.returncode == 0, res.stderr[-3000:]
    sizes = [int(m) for m in re.findall(r"mixed_attention_kernel\w*.*?\n.*?LDS Size \[bytes/block\]: (\d+)",
                                        res.stderr, flags=re.S)]
    if not sizes:  # remarks printed in another order: take every LDS size line of the file
        sizes = [int(m) for m in re.findall(r"LDS Size \[bytes/block\]: (\d+)", res.stderr)]
    assert sizes
    k_max_seqs = 1024  # kMaxSeqs: the ABI's batch limit for cie_mixed_attention
    plan = k_max_seqs * 8 + (4 * k_max_seqs + k_max_seqs + 1) * 4
    for static in sizes:
        assert static + plan <= 160 * 1024, (static, plan)
