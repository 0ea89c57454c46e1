"""Build libcie_paged.so (the gfx950 HIP kernels + C ABI) in-tree with hipcc.

The library is compiled straight from ``csrc/*.hip`` for gfx950 only; the built
``.so`` sits next to this file so it travels with the source tree.  Objects go
to ``_build/`` and the final link replaces the library atomically.

bench.py's measurement helpers (``csrc/bench/``) build into a separate
``libcie_bench.so`` (``build_bench``); the product library never contains them.

Tuning variants (the kernels' ``CIE_*`` build-time settings) build elsewhere:
``python -m custom_inference_engine_amd._build -D CIE_DECODE_TRACE=1 --out DIR``
writes ``DIR/libcie_paged.so``, which ``bench.py --lib`` times; the package
itself loads only the in-tree library.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_NAME = "libcie_paged.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
SOURCES = ("capi.hip", "kv_append.hip", "paged_decode.hip", "mixed_attention.hip")
# bench.py's measurement helpers: a library of their own, never linked into the product
BENCH_SOURCES = ("bench/gather_probe.hip",)
BENCH_LIB_PATH = os.path.join(PKG_DIR, "libcie_bench.so")
ARCH = "gfx950"

# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 in device code.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # no kernel produces NaN (masked scores are -inf and the running max is
    # always finite): lets max trees use v_max3 without canonicalizing moves
    "-fno-honor-nans",
    "-munsafe-fp-atomics",
    # kernel-argument preloading: a kernel's first 3 scalar arguments arrive
    # in SGPRs with the wave (the code object keeps a prologue that loads them
    # on firmware without preloading).  decode_kernel passes the pointers its
    # first loads need there, so they do not wait for the argument load.
    "-mllvm", "-amdgpu-kernarg-preload-count=3",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the HIP toolchain is required to build")
    return path


def _compile(src: str, verbose: bool, obj_dir: str = BUILD_DIR, defines: tuple = ()) -> str:
    obj = os.path.join(obj_dir, os.path.splitext(src)[0].replace("/", "_") + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *(f"-D{d}" for d in defines), "-I", INCLUDE, "-I", CSRC, "-c",
           os.path.join(CSRC, src), "-o", obj, "-Rpass-analysis=kernel-resource-usage"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    noise = "is not a recognized feature for this target"
    lines = [l for l in (res.stdout + res.stderr).splitlines() if noise not in l]
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n" + "\n".join(lines))
    # Hot kernels must stay in registers: any scratch use is a build error
    # (phase-trace builds excepted: their stamps are diagnostics).
    spills = [l for l in lines if "ScratchSize [bytes/lane]:" in l and not l.rstrip().endswith(": 0")
              and "ScratchSize [bytes/lane]: 0 " not in l]
    tracing = any(d.startswith(("CIE_MIXED_TRACE", "CIE_DECODE_TRACE")) for d in defines)
    if spills and not tracing:
        raise RuntimeError(f"{src}: kernel uses scratch memory (register spill):\n" + "\n".join(spills))
    msg = "\n".join(l for l in lines if "remark:" not in l)
    if verbose and msg.strip():
        print(msg, flush=True)
    return obj


def _link(objs: list, lib_path: str, verbose: bool) -> str:
    tmp = lib_path + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, lib_path)
    return lib_path


def build(verbose: bool = False, defines: tuple = (), out_dir: str | None = None) -> str:
    """Compile every HIP source for gfx950 and link ``libcie_paged.so`` (in-tree, or a
    tuning variant with extra ``NAME=VALUE`` defines into ``out_dir``)."""
    if (defines or out_dir) and not out_dir:
        raise ValueError("a build with extra defines needs its own out_dir")
    obj_dir = os.path.join(out_dir, "_build") if out_dir else BUILD_DIR
    lib_path = os.path.join(out_dir, LIB_NAME) if out_dir else LIB_PATH
    os.makedirs(obj_dir, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose, obj_dir, tuple(defines)), SOURCES))
    return _link(objs, lib_path, verbose)


def build_bench(verbose: bool = False) -> str:
    """Compile bench.py's measurement helpers into ``libcie_bench.so`` (in-tree)."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    objs = [_compile(s, verbose, BUILD_DIR) for s in BENCH_SOURCES]
    return _link(objs, BENCH_LIB_PATH, verbose)


if __name__ == "__main__":
    import argparse

    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("-v", action="store_true", help="print the compiler commands")
    ap.add_argument("-D", dest="defines", action="append", default=[], metavar="NAME=VALUE",
                    help="a CIE_* build setting (variant builds need --out)")
    ap.add_argument("--out", default=None, help="directory of a variant build")
    a = ap.parse_args()
    print(build(verbose=a.v, defines=tuple(a.defines), out_dir=a.out))
    if not a.out:
        print(build_bench(verbose=a.v))
