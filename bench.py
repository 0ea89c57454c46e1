"""Benchmark of the paged GQA decode hot path on one MI355X.

Headline (BASELINE.json metric): one decode *call* = KV append of the new token
+ split-KV GQA decode (load + merge) for one layer, at B=32, kv_len=4096 prior
(4097 attended), H_q=14, H_kv=2, D=64, page_size 16, fp16.  The layer rotates
over R distinct per-layer pools (R * pool bytes >= 512 MiB) so the 256 MB
Infinity Cache cannot serve repeat reads.  Calls are captured in a hipGraph
(R calls per graph, as a decode step walks the layers) and replayed.

Prints ONE JSON line.  ``value`` = algorithmic GB/s of a call (higher is
better); ``us_per_call`` is the same measurement as a time.  A call is one
kernel launch (the KV append fused into the decode), so ``roofline`` rates that
kernel: its per-launch time from HIP events on the stream it runs on, against
8 TB/s.  The two-launch path (append kernel + decode op) is timed beside it.  ``cpu_baseline`` times the CPU oracle
(the reference's semantics: torch gather + SDPA in fp32, numpy append) on
this host on a bounded sample of the same workload.

    python bench.py [--steps K] [--warmup W] [--config 2|3|4|5|6] [--no-cpu-baseline]
    python bench.py --copy-calib      # plain copy kernel for rocprofv3 counter scaling
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "paged GQA decode µs/call + HBM GB/s (% of peak) at B=32 kv_len=4096"
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
# HBM bytes per launch of the measured kernel, from rocprofv3 FETCH_SIZE x 2.0 +
# WRITE_SIZE (scale factors from a plain 256 MiB copy), committed under profiles/
TRAFFIC_BYTES = {
    2: (70_906_880, "profiles/hbm_traffic_decode_config2.md"),
    3: (39_666_586, "profiles/mixed_attention_config3.md"),
}
HBM_PEAK_GBPS = 8000.0
PLAN_LAYERS = 24  # decode calls per step plan: the layers of config 5's model
MIN_ROTATION_BYTES = 512 << 20


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=800, help="calls timed: exactly K, recorded in one graph (above 4,096, the R-call rotation is replayed and K rounds up to a multiple of R)")
    ap.add_argument("--warmup", type=int, default=80)
    ap.add_argument("--config", type=int, default=2, choices=(2, 3, 4, 5, 6),
                    help="6: the reference feature bench's mixed shape, beside its published times")
    ap.add_argument("--splits", type=int, default=None, help="KV splits (default: the library's policy)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="time eager launches instead of graph replay")
    ap.add_argument("--copy-calib", action="store_true")
    ap.add_argument("--variable-lengths", action="store_true",
                    help="config 2's variant: per-sequence prior lengths uniform in [512, 4096] (seed 0)")
    ap.add_argument("--probe-cus", action="store_true",
                    help="gather-probe rate of the decode call's volume on 256 / 128 / 64 CUs (per-CU read limit)")
    ap.add_argument("--repeats", type=int, default=5)
    ap.add_argument("--kernels", action="store_true",
                    help="per-launch times of the append kernels (decode B=32, token T=1052, fused "
                         "QKV-split + RoPE T=1052) and of the rope-mode decode at config 2")
    ap.add_argument("--trace-decode", action="store_true",
                    help="phase trace of one config-2 call; needs a trace build of the library "
                         "(python -m custom_inference_engine_amd._build -D CIE_DECODE_TRACE --out DIR, "
                         "then --lib DIR/libcie_paged.so)")
    ap.add_argument("--trace-planned", action="store_true",
                    help="with --trace-mixed / --trace-decode: trace planned launches (the step's plan made once)")
    ap.add_argument("--trace-mixed", action="store_true",
                    help="per-item phase trace of one config-3 mixed launch (--config 6: the feature "
                         "bench's B = 1 shape); needs a trace build (-D CIE_MIXED_TRACE, then --lib)")
    ap.add_argument("--lib", default=None, metavar="PATH",
                    help="time this build of libcie_paged.so instead of the in-tree one (a trace or "
                         "tuning build written by python -m custom_inference_engine_amd._build -D NAME=VALUE "
                         "--out DIR); the package itself only ever loads the in-tree library")
    ap.add_argument("--trace-out", default=None, metavar="PATH",
                    help="with --trace-mixed: also write every item's stamps to PATH as JSON")
    ap.add_argument("--mixed-part", choices=("all", "prefill", "decode", "long-prefill"), default="all",
                    help="config 3: time only its prefill chunks or only its decode rows; long-prefill: "
                         "4 sequences x 2,048 new tokens on no prior (a compute-heavy prefill, for the "
                         "MFMA counters of large tiles; no reference counterpart)")
    ap.add_argument("--step-modules", action="store_true",
                    help="config 5's model: one mixed step (8 sequences x 64 new tokens over 512 cached, "
                         "token bucket 512) through the eager, full-graph and piecewise step modules")
    return ap.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Layer:
    """One layer's pools + the step inputs of a decode call."""

    def __init__(self, kp, vp, q, k_new, v_new):
        self.kp, self.vp, self.q, self.k_new, self.v_new = kp, vp, q, k_new, v_new


def build_layers(case, dev, R: int, seed: int = 1):
    """Layer 0 = the seeded oracle case; layers 1..R-1 = distinct random pools of the same shape."""
    layers = [Layer(case.k_pool.to(dev), case.v_pool.to(dev), case.q.to(dev), case.k_new.to(dev),
                    case.v_new.to(dev))]
    g = torch.Generator(device=dev).manual_seed(seed)

    def rnd(t):
        return (torch.randn(t.shape, generator=g, device=dev) * 0.5).half()

    for _ in range(1, R):
        layers.append(Layer(rnd(case.k_pool), rnd(case.v_pool), rnd(case.q), rnd(case.k_new),
                            rnd(case.v_new)))
    return layers


MAX_GRAPH_CALLS = 4096


def time_calls(fn_list, steps: int, warmup: int, use_graph: bool, repeats: int) -> tuple[float, int]:
    """Median over repeats of the per-call time (us) of `steps` calls of fn_list, round-robin.

    With graphs, one hipGraph records a timed region's calls — exactly `steps`
    of them, rotating over fn_list, up to MAX_GRAPH_CALLS; beyond that
    fn_list is recorded once and replayed (steps rounded up to a multiple of
    its length).  Before every timed region the same work runs once untimed,
    so the GPU is busy while the host records the start event and enqueues
    the timed replays: the region never waits on the host's graph launch.
    Returns (us per call, calls timed per region)."""
    R = len(fn_list)
    if use_graph and steps <= MAX_GRAPH_CALLS:
        seq, reps = [fn_list[i % R] for i in range(steps)], 1
    else:
        seq, reps = fn_list, max(1, -(-steps // R))
        steps = reps * R
    stream = torch.cuda.current_stream()

    def run_all():
        for f in seq:
            f()

    if use_graph:
        from custom_inference_engine_amd.graphs import StepGraph

        body = StepGraph(run_all).replay
    else:
        body = run_all
    for _ in range(max(1, -(-warmup // len(seq)))):
        body()
    torch.cuda.synchronize()
    times = []
    for _ in range(repeats):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        body()  # untimed lead: keeps the GPU busy while the timed region is enqueued
        start.record(stream)
        for _ in range(reps):
            body()
        end.record(stream)
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end) * 1e3 / steps)
    return statistics.median(times), steps


def cpu_baseline(case, budget_s: float = 20.0, max_runs: int = 7):
    """The oracle (reference semantics) on this host's cores: numpy append + torch gather/SDPA fp32."""
    from oracle import paged_attention as ref

    n_cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(n_cores)

    def one():
        kp, vp = case.k_pool.clone(), case.v_pool.clone()
        t0 = time.perf_counter()
        ref.append_decode(kp, vp, case.k_new, case.v_new, case.slot_ids, case.lens_pool, case.block_table)
        out = ref.decode_attention(case.q, kp, vp, case.attended, case.slot_ids, case.block_table)
        return time.perf_counter() - t0, out

    runs, spent = [], 0.0
    for i in range(2 + max_runs):
        dt, out = one()
        spent += dt
        if i >= 2:
            runs.append(dt)
        if len(runs) >= 5 and spent > budget_s:
            break
    return statistics.median(runs) * 1e6, len(runs), torch.get_num_threads(), out


_bench_lib = None


def bench_lib():
    """libcie_bench.so: bench-only measurement kernels, kept out of the product
    library (built by the package's build_bench(), here if it is missing)."""
    global _bench_lib
    if _bench_lib is None:
        import ctypes

        from custom_inference_engine_amd import _build

        if not os.path.exists(_build.BENCH_LIB_PATH):
            _build.build_bench()
        lib = ctypes.CDLL(_build.BENCH_LIB_PATH)
        p, i64 = ctypes.c_void_p, ctypes.c_int64
        lib.cie_bench_gather_read.restype = ctypes.c_int
        lib.cie_bench_gather_read.argtypes = [p, p, i64, i64, i64, p, p]
        lib.cie_bench_gather_read_waves.restype = ctypes.c_int
        lib.cie_bench_gather_read_waves.argtypes = [p, p, i64, i64, ctypes.c_int, p, p]
        _bench_lib = lib
    return _bench_lib


def gather_ceiling(dev, nbytes: int, steps: int, warmup: int, repeats: int, chunk: int = 2048,
                   region_bytes: int = 1 << 30, grid: tuple[int, int] | None = None):
    """HBM ceiling of the paged access pattern on this box: the probe kernel reads
    the same byte volume as one decode call as shuffled chunk-sized pieces of a
    1 GiB region (R disjoint chunk lists rotate, so the 256 MB MALL cannot help).
    grid = (workgroups, waves per workgroup) runs the 2 KiB probe on that grid."""
    from custom_inference_engine_amd import _native

    lib = bench_lib()
    region = torch.ones(region_bytes, dtype=torch.uint8, device=dev)
    n_region = region.numel() // chunk
    n = nbytes // chunk
    R = max(1, min(8, n_region // n))
    perm = torch.randperm(n_region, generator=torch.Generator().manual_seed(7))
    lists = [perm[i * n:(i + 1) * n].to(torch.int32).to(dev) for i in range(R)]
    sink = torch.zeros(1, dtype=torch.int32, device=dev)

    def f(i):
        def g():
            if grid is not None:
                rc = lib.cie_bench_gather_read_waves(region.data_ptr(), lists[i].data_ptr(), n, grid[0],
                                                     grid[1], sink.data_ptr(), _native.stream_handle(dev))
            else:
                rc = lib.cie_bench_gather_read(region.data_ptr(), lists[i].data_ptr(), n, chunk, 2048,
                                               sink.data_ptr(), _native.stream_handle(dev))
            if rc != 0:
                raise RuntimeError(f"cie_bench_gather_read failed: status {rc}")
        return g

    us, _ = time_calls([f(i) for i in range(R)], steps, warmup, True, repeats)
    del region
    return us, n * chunk


def bench_kernels(args):
    """Per-launch times (one hipGraph of at least 128 launches over rotating inputs) of
    the kernels the drop-in runs besides the headline call: the standalone KV
    appends (decode mode at config 2's B = 32; token mode and the fused
    QKV-split + RoPE + append at config 3's T = 1052) and the rope-mode decode
    (QKV split + RoPE + append + split-KV decode in one launch) at config 2.
    A one-element torch add is timed beside them: the floor of a launch that
    loads and stores one value."""
    import custom_inference_engine_amd as cie
    from oracle import inputs

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev).manual_seed(3)

    def rnd(*shape):
        return (torch.randn(shape, generator=gen, device=dev) * 0.5).half()

    def timed(fns):
        # graphs of >= 128 launches: a replay of a few microsecond-scale kernels
        # is shorter than the host's graph launch, which would then be timed
        fns = fns * max(1, -(-128 // len(fns)))
        return time_calls(fns, max(args.steps, 4 * len(fns)), args.warmup, True, args.repeats)

    out = {}
    one = torch.zeros(1, device=dev)
    us, _ = timed([lambda: one.add_(1.0)])
    out["floor_one_element_add"] = us
    log(f"one-element add (launch floor): {us:.2f} us")

    case2 = inputs.config2(seed=0)
    c2 = case2.to(dev)
    R = max(1, -(-MIN_ROTATION_BYTES // (2 * case2.k_pool.numel() * 2)))
    pools = [(c2.k_pool.clone(), c2.v_pool.clone()) for _ in range(R)]
    us, _ = timed([lambda kp=kp, vp=vp: cie.kv_append_decode(kp, vp, c2.k_new, c2.v_new, c2.slot_ids,
                                                             c2.lens_pool, c2.block_table)
                   for kp, vp in pools])
    out["kv_append_decode_b32"] = us
    log(f"kv_append_kernel<8,true> (decode append, B={case2.B}): {us:.2f} us")
    qkvs = [rnd(1, case2.B, (14 + 4) * 64) for _ in range(R)]
    cos, sin = rnd(1, case2.B, 64), rnd(1, case2.B, 64)
    us, _ = time_calls([lambda i=i: cie.decode_qkv_rope_gqa_attention(qkvs[i], cos, sin, pools[i][0], pools[i][1],
                                                                      c2.lens_pool, c2.slot_ids, c2.block_table,
                                                                      num_heads=14)
                        for i in range(R)], args.steps, args.warmup, True, args.repeats)  # ~17 us each
    out["decode_rope_config2"] = us
    log(f"decode_kernel<64,4,true,true> (rope mode, config 2): {us:.2f} us")
    del pools

    case3 = inputs.config3(seed=0)
    c3 = case3.to(dev)
    T = case3.T
    pools = [(c3.k_pool.clone(), c3.v_pool.clone()) for _ in range(4)]
    us, _ = timed([lambda kp=kp, vp=vp: cie.kv_append_tokens(kp, vp, c3.k_new, c3.v_new, c3.pages, c3.offsets)
                   for kp, vp in pools])
    out["kv_append_tokens_t1052"] = us
    log(f"kv_append_kernel<8,false> (token append, T={T}): {us:.2f} us")
    qkv3 = [rnd(1, T, (14 + 4) * 64) for _ in range(4)]
    cos3, sin3 = rnd(1, T, 64), rnd(1, T, 64)
    us, _ = timed([lambda i=i: cie.append_tokens_qkv_rope(qkv3[i], cos3, sin3, pools[i][0], pools[i][1],
                                                          c3.pages, c3.offsets, num_heads=14)
                   for i in range(4)])
    out["qkv_rope_append_t1052"] = us
    log(f"qkv_rope_append_kernel (QKV split + RoPE + append, T={T}): {us:.2f} us")
    print(json.dumps({"metric": "per-launch us of the append kernels and the rope-mode decode",
                      "unit": "us", "higher_is_better": False,
                      **{k: round(v, 3) for k, v in out.items()}}), flush=True)


def trace_decode(args):
    """Phase trace of one config-2 call (append fused; --variable-lengths: its variant) after R warm calls.

    A trace build stamps s_memrealtime (100 MHz) into LDS at phase boundaries
    and each workgroup copies its stamps out as it exits; printed: per phase
    the min / median / max over workgroups (µs from the first workgroup's
    start), the loop end by XCD, and per split and wave the first step and
    the loop end."""
    import collections
    import ctypes

    import custom_inference_engine_amd as cie
    from custom_inference_engine_amd import _native
    from oracle import inputs

    lib = _native.load()
    if not hasattr(lib, "cie_decode_trace_buffer"):
        raise SystemExit("--trace-decode needs a trace build (see --help)")
    lib.cie_decode_trace_buffer.argtypes = [ctypes.c_void_p]
    dev = torch.device("cuda:0")
    case = inputs.config2(seed=0, fixed=not args.variable_lengths)
    c = case.to(dev)
    S = args.splits or cie.attn.core.default_decode_splits(case.B, 2, dev)
    W, slots = 4, 24
    R = max(1, -(-MIN_ROTATION_BYTES // (2 * case.k_pool.numel() * 2)))
    pools = [(c.k_pool.clone(), c.v_pool.clone()) for _ in range(R)]
    plan = (cie.decode_plan(pools[0][0], c.lens_pool, c.slot_ids, c.block_table, append=True, num_programs=S)
            if args.trace_planned else None)
    n_wg = plan.numel() // cie.attn.core.PLAN_WORDS_PER_WORKGROUP if plan is not None else case.B * 2 * S
    buf = torch.zeros(max(n_wg, case.B * 2 * S) * slots, dtype=torch.int64, device=dev)
    if lib.cie_decode_trace_buffer(buf.data_ptr()) != 0:
        raise SystemExit("cie_decode_trace_buffer failed")
    for it in range(3 * R):
        kp, vp = pools[it % R]
        buf.zero_()
        cie.decode_append_gqa_attention(c.q, kp, vp, c.k_new, c.v_new, c.lens_pool, c.slot_ids,
                                        c.block_table, num_programs=None if plan is not None else S, plan=plan)
    torch.cuda.synchronize()
    lib.cie_decode_trace_buffer(None)
    t = buf.view(-1, slots).cpu()
    t = t[t[:, 0] != 0]  # workgroups that ran (a plan may leave some idle)
    t0 = t[:, 0].min().item()

    def us(v):
        return (v - t0) / 100.0

    phases = {0: "workgroup start", 1: "slot -> pages + length + Q known", 8: "fold barrier",
              9: "partials issued", 10: "arrival atomic returned", 4: "merge end (last arriver)"}
    for k, name in phases.items():
        v = [us(x) for x in t[:, k].tolist() if x]
        if v:
            print(f"{name:34s} min {min(v):6.2f}  median {statistics.median(v):6.2f}  max {max(v):6.2f}")
    ends = [us(max(t[r, 16:16 + W].tolist())) for r in range(t.shape[0])]
    print(f"{'slowest wave of the workgroup ends':34s} min {min(ends):6.2f}  median "
          f"{statistics.median(ends):6.2f}  max {max(ends):6.2f}")
    by_xcd = collections.defaultdict(list)
    for r in range(t.shape[0]):
        by_xcd[int(t[r, 6].item()) & 0xF].append(ends[r])
    print("loop end by XCD (median/max): " + "  ".join(
        f"{x}:{statistics.median(v):.2f}/{max(v):.2f}" for x, v in sorted(by_xcd.items())))
    for sp in range(0 if plan is not None else S):
        rows = [r for r in range(t.shape[0]) if r % S == sp]
        for w in range(W):
            first = [us(t[r, 20 + w].item()) for r in rows if t[r, 20 + w].item()]
            end = [us(t[r, 16 + w].item()) for r in rows]
            print(f"split {sp} wave {w}: first step done {statistics.median(first):6.2f}  "
                  f"loop end median {statistics.median(end):6.2f} max {max(end):6.2f}")


def trace_mixed(args):
    """Per-item phase trace of one config-3 mixed launch (``--mixed-part`` applies).

    Each work item's stamps (µs from the first item's start): start, tile
    lookup done, Q staged, key loop done, fold done, end (plus merge for the
    last chunk of a split tile).  Printed: the span, the critical item, and
    per item class (column tiles x chunked) the median phase durations."""
    import ctypes

    import custom_inference_engine_amd as cie
    from custom_inference_engine_amd import _native
    from oracle import inputs

    lib = _native.load()
    if not hasattr(lib, "cie_mixed_trace_buffer"):
        raise SystemExit("--trace-mixed needs a trace build (see --help)")
    lib.cie_mixed_trace_buffer.argtypes = [ctypes.c_void_p]
    dev = torch.device("cuda:0")
    case = inputs.config3(seed=0)
    max_seqlen = 256
    if args.config == 6:  # the feature bench's B = 1 shape: 128 rows on 256 cached tokens
        case, max_seqlen = inputs.make_case([256], [128], seed=1), 128
    elif args.mixed_part != "all":
        prior, new = case.kv_lens.tolist(), case.new_lens.tolist()
        keep = [i for i, n in enumerate(new) if (n > 1) == (args.mixed_part == "prefill")]
        case = inputs.make_case([prior[i] for i in keep], [new[i] for i in keep], seed=0)
    c = case.to(dev)
    R = 8
    pools = [(c.k_pool.clone(), c.v_pool.clone()) for _ in range(R)]
    buf = torch.zeros(2 * 4096 * 16, dtype=torch.int64, device=dev)
    if lib.cie_mixed_trace_buffer(buf.data_ptr()) != 0:
        raise SystemExit("cie_mixed_trace_buffer failed")
    plan = (cie.mixed_plan(pools[0][0], c.cu_seqlens, c.kv_lens, c.slot_ids, c.block_table, max_seqlen, case.T,
                           case.q.shape[2]) if args.trace_planned else None)
    for it in range(3 * R):
        kp, vp = pools[it % R]
        buf.zero_()
        cie.mixed_gqa_attention(c.q, kp, vp, max_seqlen, c.cu_seqlens, c.kv_lens, c.slot_ids, c.block_table,
                                plan=plan)
    torch.cuda.synchronize()
    lib.cie_mixed_trace_buffer(None)
    t = buf.view(2, 4096, 16).cpu()
    valid = t[:, :, 0] != 0
    t0 = t[:, :, 0][valid].min().item()

    def us(x):
        return (x - t0) / 100.0

    items = []
    for g in range(2):
        for i in range(4096):
            if not valid[g, i]:
                continue
            r = t[g, i].tolist()
            info = r[5]
            items.append(dict(g=g, item=i, start=us(r[0]), lookup=us(r[1]), q=us(r[9]), loop=us(r[8]),
                              wave_loops=[us(x) if x else None for x in r[10:14]], wg=r[14],
                              wg_start=us(r[15]) if r[15] else None,
                              fold=us(r[2]), end=us(r[3]), merge=us(r[4]) if r[4] else None,
                              nct=info // 1000000, nch=(info // 10000) % 100, ktiles=info % 10000,
                              seq=r[7] // 1000, qt=r[7] % 1000))
    span = max(x["end"] for x in items)
    crit = max(items, key=lambda x: x["end"])
    starts = [x["wg_start"] for x in items if x["wg_start"] is not None]
    print(f"items {len(items)}, span {span:.2f} us; planning done (median over workgroups) "
          f"{statistics.median(us(t[g, i, 6].item()) for g in range(2) for i in range(4096) if t[g, i, 6]):.2f} us; "
          f"workgroup starts {min(starts):.2f} .. {max(starts):.2f} us (median {statistics.median(starts):.2f})")
    print("critical item: " + ", ".join(f"{k} {v:.2f}" if isinstance(v, float) else f"{k} {v}"
                                        for k, v in crit.items()))
    print(f"{'class':18s} {'n':>4s} {'start':>6s} {'lookup':>7s} {'Q':>6s} {'loop':>7s} {'fold':>6s} "
          f"{'end':>6s} {'end max':>8s}  (µs; start absolute, the rest after the item's start)")
    for nct in (1, 2, 3, 4):
        for chunked in (False, True):
            sel = [x for x in items if x["nct"] == nct and (x["nch"] > 1) == chunked]
            if not sel:
                continue
            med = lambda k: statistics.median(x[k] - x["start"] for x in sel)
            print(f"{nct} col tile(s){' chunked' if chunked else '':8s} {len(sel):4d} "
                  f"{statistics.median(x['start'] for x in sel):6.2f} {med('lookup'):7.2f} {med('q'):6.2f} "
                  f"{med('loop'):7.2f} {med('fold'):6.2f} {med('end'):6.2f} "
                  f"{max(x['end'] - x['start'] for x in sel):8.2f}")
    if args.trace_out:
        with open(args.trace_out, "w") as f:
            json.dump(items, f)
    late = sorted(items, key=lambda x: -x["end"])[:8]
    print("latest items (seq, tile, col tiles, chunks, key tiles: start -> end):")
    for x in late:
        print(f"  seq {x['seq']} tile {x['qt']} ct {x['nct']} ch {x['nch']} kt {x['ktiles']}: "
              f"{x['start']:.2f} -> {x['end']:.2f} (loop {x['loop'] - x['start']:.2f})")


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def copy_calibration(args):
    """A plain device copy of known size, for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE."""
    n = 256 << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda").random_()
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "launches": 5}), flush=True)


def probe_cus(args):
    """The decode call's K/V volume read as shuffled 2 KiB chunks by the whole chip
    (256 workgroups of 4 waves, one per CU) and by fewer CUs with more waves each
    (128 x 8, 64 x 16): whether a (sequence, kv head) can be read by one CU, with no
    split and no merge (config 2 has 64 of them)."""
    dev = torch.device("cuda:0")
    nbytes = 32 * 2 * 4097 * 256  # config 2's K and V bytes
    for wg, waves in ((256, 4), (128, 8), (64, 16)):
        us, moved = gather_ceiling(dev, nbytes, 400, 40, 3, 2048, 1 << 30, grid=(wg, waves))
        print(json.dumps({"probe_bytes": moved, "workgroups": wg, "waves_per_workgroup": waves,
                          "us": round(us, 2), "TBps": round(moved / us / 1e6, 3),
                          "GBps_per_cu": round(moved / us / 1e3 / wg, 1)}), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); this build's hot path is "
              "single-GPU and launches no collectives.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(2)
    if args.lib:
        from custom_inference_engine_amd import _native

        _native.LIB_PATH = os.path.abspath(args.lib)
    if args.copy_calib:
        return copy_calibration(args)
    if args.probe_cus:
        return probe_cus(args)
    if args.kernels:
        return bench_kernels(args)
    if args.trace_decode:
        return trace_decode(args)
    if args.trace_mixed:
        return trace_mixed(args)

    import custom_inference_engine_amd as cie
    from custom_inference_engine_amd import _native
    from oracle import inputs, paged_attention as ref

    _native.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.config == 3:
        return bench_mixed(args, cie, inputs, ref, dev)
    if args.step_modules:
        return bench_step_modules(args, cie, dev)
    if args.config == 5:
        return bench_model(args, cie, dev)
    if args.config == 6:
        return bench_feature_shapes(args, cie, inputs, ref, dev)
    case = (inputs.config2(seed=0, fixed=not args.variable_lengths) if args.config == 2
            else inputs.config4(seed=0))
    splits = args.splits or (case.meta.get("n_splits") if args.config == 4 else None)
    log(f"config {args.config}: B={case.B} attend={int(case.attended[0])} pool pages={case.k_pool.shape[0]}")

    pool_bytes = 2 * case.k_pool.numel() * 2
    R = max(1, -(-MIN_ROTATION_BYTES // pool_bytes))
    layers = build_layers(case, dev, R)
    c = case.to(dev)
    slot_ids, lens_pool, bt = c.slot_ids, c.lens_pool, c.block_table
    attended = (lens_pool[slot_ids] + 1).contiguous()
    log(f"rotation: {R} layer pools x {pool_bytes / 2**20:.1f} MiB = {R * pool_bytes / 2**20:.0f} MiB")

    outs = [None] * R

    def call_fused(i):
        L = layers[i]

        def f():
            outs[i] = cie.decode_append_gqa_attention(L.q, L.kp, L.vp, L.k_new, L.v_new, lens_pool,
                                                      slot_ids, bt, num_programs=splits)
        return f

    def call_two_launch(i):
        L = layers[i]

        def f():
            cie.kv_append_decode(L.kp, L.vp, L.k_new, L.v_new, slot_ids, lens_pool, bt)
            outs[i] = cie.decode_gqa_attention(L.q, L.kp, L.vp, attended, slot_ids, bt, num_programs=splits)
        return f

    def decode_only(i):
        L = layers[i]

        def f():
            outs[i] = cie.decode_gqa_attention(L.q, L.kp, L.vp, attended, slot_ids, bt, num_programs=splits)
        return f

    # parity spot check of layer 0 (both paths) against the oracle before timing
    kp0, vp0 = case.appended_pools()
    want = ref.decode_attention(case.q, kp0, vp0, case.attended, case.slot_ids, case.block_table)
    for name, mk in (("fused", call_fused), ("two-launch", call_two_launch)):
        layers[0].kp.copy_(c.k_pool)
        layers[0].vp.copy_(c.v_pool)
        mk(0)()
        torch.cuda.synchronize()
        err = (outs[0][0].float().cpu() - want).abs().max().item()
        pool_ok = torch.equal(layers[0].kp.cpu().view(torch.int16), kp0.view(torch.int16)) and \
            torch.equal(layers[0].vp.cpu().view(torch.int16), vp0.view(torch.int16))
        log(f"parity ({name}): max abs err {err:.2e}, append bit-exact {pool_ok}")
        if err > 2e-3 or not pool_ok:
            raise SystemExit(f"parity check failed ({name}: err {err}, append exact {pool_ok})")

    use_graph = not args.no_graph
    us_call, steps = time_calls([call_fused(i) for i in range(R)], args.steps, args.warmup, use_graph,
                                args.repeats)
    log(f"call, fused append + decode (1 launch): {us_call:.2f} us")
    us_two, _ = time_calls([call_two_launch(i) for i in range(R)], args.steps, args.warmup, use_graph,
                           args.repeats)
    log(f"call, append + decode op (2 launches): {us_two:.2f} us")
    us_eager, _ = time_calls([call_fused(i) for i in range(R)], max(R, args.steps // 4), R, False, 3)
    log(f"call, fused, eager launches: {us_eager:.2f} us")
    us_dec, _ = time_calls([decode_only(i) for i in range(R)], args.steps, args.warmup, use_graph, args.repeats)
    log(f"decode op alone (1 launch): {us_dec:.2f} us")
    # the Qwen2 drop-in's default decode launch: QKV split + RoPE + append +
    # split-KV decode from the fused projection's output row (same pools)
    qkv_rows = [torch.cat([L.q.reshape(1, case.B, -1), L.k_new.reshape(1, case.B, -1),
                           L.v_new.reshape(1, case.B, -1)], dim=-1).contiguous() for L in layers]
    gcs = torch.Generator(device=dev).manual_seed(3)
    cos_t = torch.rand((1, case.B, 64), generator=gcs, device=dev).half()
    sin_t = torch.rand((1, case.B, 64), generator=gcs, device=dev).half()

    def call_rope(i):
        L = layers[i]
        return lambda: cie.decode_qkv_rope_gqa_attention(qkv_rows[i], cos_t, sin_t, L.kp, L.vp, lens_pool,
                                                         slot_ids, bt, num_heads=14, num_programs=splits)
    us_rope, _ = time_calls([call_rope(i) for i in range(R)], args.steps, args.warmup, use_graph,
                            args.repeats)
    log(f"call, QKV split + RoPE + append + decode (the drop-in's launch): {us_rope:.2f} us")
    # Planned calls: a decode step makes one plan (decode_plan) for all of its
    # layers, so the timed sequence launches the plan once per PLAN_LAYERS
    # calls (Qwen2.5-0.5B has 24 layers), inside the timed region.
    plan_holder = [None]

    def make_plan():
        plan_holder[0] = cie.decode_plan(layers[0].kp, lens_pool, slot_ids, bt, append=True,
                                         num_programs=splits)

    def call_planned(k):
        L = layers[k % R]

        def f():
            if k == 0:
                make_plan()
            outs[k % R] = cie.decode_append_gqa_attention(L.q, L.kp, L.vp, L.k_new, L.v_new, lens_pool,
                                                          slot_ids, bt, plan=plan_holder[0])
        return f
    make_plan()
    torch.cuda.synchronize()
    layers[0].kp.copy_(c.k_pool)
    layers[0].vp.copy_(c.v_pool)
    call_planned(0)()  # layer 0, with the plan made as a step's first call makes it
    torch.cuda.synchronize()
    err_p = (outs[0][0].float().cpu() - want).abs().max().item()
    log(f"parity (planned): max abs err {err_p:.2e}")
    if err_p > 2e-3:
        raise SystemExit(f"parity check failed (planned: err {err_p})")
    us_planned, _ = time_calls([call_planned(k) for k in range(PLAN_LAYERS)], args.steps, args.warmup,
                               use_graph, args.repeats)
    log(f"call, planned fused append + decode (1 plan per {PLAN_LAYERS} calls): {us_planned:.2f} us")

    def call_rope_planned(k):
        L = layers[k % R]

        def f():
            if k == 0:
                make_plan()
            cie.decode_qkv_rope_gqa_attention(qkv_rows[k % R], cos_t, sin_t, L.kp, L.vp, lens_pool, slot_ids,
                                              bt, num_heads=14, plan=plan_holder[0])
        return f
    us_rope_planned, _ = time_calls([call_rope_planned(k) for k in range(PLAN_LAYERS)], args.steps,
                                    args.warmup, use_graph, args.repeats)
    log(f"call, planned QKV split + RoPE + append + decode (1 plan per {PLAN_LAYERS} calls): "
        f"{us_rope_planned:.2f} us")

    us_default = None
    if splits is not None and args.splits is None:
        # the config states its split count; the library's own choice beside it
        def call_default(i):
            L = layers[i]
            return lambda: cie.decode_append_gqa_attention(L.q, L.kp, L.vp, L.k_new, L.v_new, lens_pool,
                                                           slot_ids, bt)
        us_default, _ = time_calls([call_default(i) for i in range(R)], args.steps, args.warmup, use_graph,
                                   args.repeats)
        log(f"call, fused, the library's default split count "
            f"({cie.attn.core.default_decode_splits(case.B, 2, dev)}): {us_default:.2f} us")

    attended_list = case.attended.tolist()
    bytes_call = ref.decode_algorithmic_bytes(attended_list, 14, 2, 64, 16)
    gbps = bytes_call / (us_call * 1e-6) / 1e9
    us_ceil, ceil_bytes = gather_ceiling(dev, bytes_call, args.steps, args.warmup, args.repeats)
    ceil_gbps = ceil_bytes / (us_ceil * 1e-6) / 1e9
    log(f"paged-gather ceiling (probe, 2 KiB chunks): {us_ceil:.2f} us, {ceil_gbps:.0f} GB/s")

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        cpu_us, n_runs, threads, _ = cpu_baseline(case)
        cpu = {"value": round(bytes_call / (cpu_us * 1e-6) / 1e9, 3), "unit": "GB/s", "cores": threads,
               "kind": "port", "us_per_call": round(cpu_us, 1),
               "sample": f"the full headline call (append + decode, B={case.B}, attend "
                         f"{attended_list[0]}), median of {n_runs} runs after 2 warmups, "
                         f"{threads} threads on {cpu_model()}"}
        log(f"cpu baseline: {cpu_us:.0f} us/call on {threads} threads")

    wl = ("paged GQA decode call = KV append + split-KV load + merge, one layer, one launch" if args.config == 2
          else "long-context paged GQA decode call (config 4)")
    n_splits = splits or cie.attn.core.default_decode_splits(case.B, 2, dev)
    # the library's decode workgroups have 4 waves (one per SIMD) at D = 64
    waves = 4
    line = {
        "metric": METRIC if args.config == 2 else
        "long-context paged GQA decode us/call + HBM GB/s (% of peak) at B=16 kv_len=16384 (config 4)",
        "value": round(gbps, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_call / 1e3, 6),
        "us_per_call": round(us_call, 3),
        "pct_of_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 1),
        "us_per_call_eager": round(us_eager, 3),
        "us_per_call_two_launch": round(us_two, 3),
        "us_decode_op_alone": round(us_dec, 3),
        "us_per_call_qkv_rope": round(us_rope, 3),
        "us_per_call_planned": round(us_planned, 3),
        "us_per_call_qkv_rope_planned": round(us_rope_planned, 3),
        "us_per_call_default_splits": None if us_default is None else round(us_default, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 (fp32 accumulate)",
        "data": "synthetic (seeded N(0,1)*0.5 pools, shuffled pages)",
        "config": {
            "workload": wl,
            "config_id": args.config,
            "batch": case.B,
            "kv_len_prior": (int(case.kv_lens[0]) if not args.variable_lengths else
                             f"U[512, 4096] per sequence (sum {int(case.kv_lens.sum())})"),
            "attended": attended_list[0] if not args.variable_lengths else sum(attended_list),
            "heads_q": 14, "heads_kv": 2, "head_dim": 64, "page_size": 16,
            "pool_pages_per_layer": int(case.k_pool.shape[0]),
            "layer_rotation": R,
            "splits": n_splits,
            "timing": ("one hipGraph of the K timed calls rotating over the layer pools, after an untimed lead replay"
                       if use_graph and steps <= MAX_GRAPH_CALLS else
                       "hipGraph replay of the layer rotation" if use_graph else "eager launches"),
            "algorithmic_bytes_per_call": bytes_call,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": f"decode_kernel<64,{waves},true> (fused append + split-KV + merge, 1 launch/call)",
            "achieved": round(gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4),
            "us_per_launch": round(us_call, 3),
            "algorithmic_bytes_per_launch": bytes_call,
            "traffic": TRAFFIC_BYTES.get(args.config, (None, None))[0],
            "traffic_source": TRAFFIC_BYTES.get(args.config, (None, None))[1],
        },
        "paged_gather_ceiling": {
            "what": "probe kernel reading the call's byte volume as shuffled 2 KiB chunks (no math)",
            "value": round(ceil_gbps, 1), "unit": "GB/s", "us": round(us_ceil, 3),
            "frac_of_peak": round(ceil_gbps / HBM_PEAK_GBPS, 4),
            "decode_frac_of_ceiling": round(gbps / ceil_gbps, 4),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def bench_mixed(args, cie, inputs, ref, dev):
    """Config 3 (mixed chunked prefill + decode): us/call of append + mixed attention.

    ``--mixed-part prefill`` / ``decode`` time the config's 4 prefill chunks or
    its 28 decode rows alone (the same draws), e.g. to read the MFMA counters
    of the prefill tiles without the decode rows."""
    case = inputs.config3(seed=0)
    max_seqlen = case.meta["max_seqlen"]
    if args.mixed_part == "long-prefill":
        case = inputs.make_case([0] * 4, [2048] * 4, seed=0)
        max_seqlen = 2048
    elif args.mixed_part != "all":
        prior, new = case.kv_lens.tolist(), case.new_lens.tolist()
        keep = [i for i, n in enumerate(new) if (n > 1) == (args.mixed_part == "prefill")]
        case = inputs.make_case([prior[i] for i in keep], [new[i] for i in keep], seed=0)
    c = case.to(dev)
    pool_bytes = 2 * case.k_pool.numel() * 2
    R = max(1, -(-MIN_ROTATION_BYTES // pool_bytes))
    layers = build_layers(case, dev, R)
    outs = [None] * R

    def call(i):
        L = layers[i]

        def f():
            cie.kv_append_tokens(L.kp, L.vp, L.k_new, L.v_new, c.pages, c.offsets)
            outs[i] = cie.mixed_gqa_attention(L.q, L.kp, L.vp, max_seqlen, c.cu_seqlens, c.kv_lens,
                                              c.slot_ids, c.block_table)
        return f

    call(0)()
    torch.cuda.synchronize()
    want, written = ref.mixed_attention(case.q, *case.appended_pools(), case.cu_seqlens, case.kv_lens,
                                        case.slot_ids, case.block_table)
    err = (outs[0][0].float().cpu() - want)[written].abs().max().item()
    log(f"mixed parity: max abs err {err:.2e}")
    us, steps = time_calls([call(i) for i in range(R)], args.steps, args.warmup, not args.no_graph,
                           args.repeats)

    # the mixed kernel alone (the roofline's kernel), on the same rotating layers
    def mixed_only(i):
        L = layers[i]
        return lambda: cie.mixed_gqa_attention(L.q, L.kp, L.vp, max_seqlen, c.cu_seqlens, c.kv_lens,
                                               c.slot_ids, c.block_table)

    us_mix, _ = time_calls([mixed_only(i) for i in range(R)], args.steps, args.warmup, not args.no_graph,
                           args.repeats)
    log(f"config 3: {us:.2f} us/call (append + mixed), mixed kernel alone {us_mix:.2f} us/launch")
    # Planned launches: a mixed step makes one plan (mixed_plan) for all of
    # its layers, so the timed sequence launches the plan once per
    # PLAN_LAYERS calls, inside the timed region.
    us_mix_planned, err_planned = time_mixed_planned(cie, layers, c, case, max_seqlen, 14, args)
    log(f"planned: mixed kernel {us_mix_planned:.2f} us/launch (1 plan per {PLAN_LAYERS} launches), "
        f"planned == unplanned: {err_planned}")
    E = (case.kv_lens + case.new_lens).tolist()
    kv_bytes = 2 * sum(E) * 2 * 64 * 2
    qo = 2 * case.T * 14 * 64 * 2
    app = 2 * case.T * 2 * 64 * 2 * 2
    nbytes = kv_bytes + qo + app
    flops = 0
    for cc, L in zip(case.kv_lens.tolist(), case.new_lens.tolist()):
        keys = sum(cc + i + 1 for i in range(L))
        flops += 4 * 14 * 64 * keys
    print(json.dumps({
        "metric": "mixed varlen chunked prefill + decode us/call (config 3)" if args.mixed_part == "all"
        else "mixed varlen attention us/call (4 x 2,048-token prefill, no prior)"
        if args.mixed_part == "long-prefill"
        else f"mixed varlen attention us/call (config 3, its {args.mixed_part} part only)",
        "value": round(us, 3), "unit": "us/call", "higher_is_better": False, "n_gpus": 1,
        "steps": steps, "warmup": args.warmup, "ms_per_step": round(us / 1e3, 6),
        "achieved_GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
        "achieved_TFLOPs": round(flops / (us * 1e-6) / 1e12, 2),
        "us_mixed_kernel": round(us_mix, 3),
        "us_mixed_kernel_planned": round(us_mix_planned, 3),
        "dtype": "fp16 (fp32 accumulate)", "data": "synthetic",
        "config": {"workload": {"all": "config 3 mixed: 4x256-row prefill chunks + 28 decode rows",
                                "prefill": "config 3's 4x256-row prefill chunks alone",
                                "decode": "config 3's 28 decode rows alone",
                                "long-prefill": "4 sequences x 2,048 new tokens on no prior (no reference "
                                                "counterpart)"}[args.mixed_part], "T": case.T,
                   "algorithmic_bytes": nbytes, "flops": flops, "layer_rotation": R},
        "roofline": {"bound": "mfma", "kernel": "mixed_attention_kernel<64>",
                     "achieved": round(flops / (us_mix * 1e-6) / 1e12, 2), "peak": MFMA_F16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(flops / (us_mix * 1e-6) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
                     "hbm_frac": round((nbytes - app) / (us_mix * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
                     "traffic": TRAFFIC_BYTES[3][0] if args.mixed_part == "all" else None,
                     "traffic_source": TRAFFIC_BYTES[3][1] if args.mixed_part == "all" else None},
        "parity_max_abs_err": err,
    }), flush=True)


def time_mixed_planned(cie, layers, c, case, max_seqlen: int, h_q: int, args):
    """us per planned mixed launch over the rotating layers, the plan made once
    per PLAN_LAYERS launches inside the timed region; and whether layer 0's
    planned output equals its unplanned one bit for bit."""
    R = len(layers)
    holder = [None]

    def make_plan():
        holder[0] = cie.mixed_plan(layers[0].kp, c.cu_seqlens, c.kv_lens, c.slot_ids, c.block_table,
                                   max_seqlen, case.T, h_q)

    def planned(k):
        L = layers[k % R]

        def f():
            if k == 0:
                make_plan()
            cie.mixed_gqa_attention(L.q, L.kp, L.vp, max_seqlen, c.cu_seqlens, c.kv_lens, c.slot_ids,
                                    c.block_table, plan=holder[0])
        return f
    make_plan()
    L = layers[0]
    o_u = cie.mixed_gqa_attention(L.q, L.kp, L.vp, max_seqlen, c.cu_seqlens, c.kv_lens, c.slot_ids,
                                  c.block_table)
    o_p = cie.mixed_gqa_attention(L.q, L.kp, L.vp, max_seqlen, c.cu_seqlens, c.kv_lens, c.slot_ids,
                                  c.block_table, plan=holder[0])
    torch.cuda.synchronize()
    rows = int(case.cu_seqlens[-1])
    same = bool(torch.equal(o_u[0, :rows], o_p[0, :rows]))
    us, _ = time_calls([planned(k) for k in range(PLAN_LAYERS)], args.steps, args.warmup, not args.no_graph,
                       args.repeats)
    return us, same


# mixed_gqa_attention_kernel us/call at T = 128 by batch size, RTX 4070 Laptop
# (feature_bench/results/token_threshold/20261104-084454_full_graph_token_jump.json:1)
PUBLISHED_MIXED_T128 = {1: 24.09, 2: 21.14, 4: 21.41, 8: 28.80, 16: 30.67, 32: 35.09}


def bench_feature_shapes(args, cie, inputs, ref, dev, tokens: int = 128, context: int = 256):
    """The reference feature bench's mixed step (feature_bench/full_graph_token_jump.py:19-22, 48-55).

    B sequences share `tokens` new tokens (split evenly), each on `context`
    cached tokens; one layer's mixed attention (the append is timed apart in
    the reference too) with max_seqlen = the token count.  Pages here are
    shuffled (the reference's bench assigns them contiguously).  Printed beside
    the reference's published kernel times, measured on other hardware.
    """
    table = []
    for B in sorted(PUBLISHED_MIXED_T128):
        lens = [tokens // B + (1 if i < tokens % B else 0) for i in range(B)]
        case = inputs.make_case([context] * B, lens, seed=B)
        R = 8
        layers = build_layers(case, dev, R)
        c = case.to(dev)
        for L in layers:
            cie.kv_append_tokens(L.kp, L.vp, L.k_new, L.v_new, c.pages, c.offsets)
        torch.cuda.synchronize()
        o = cie.mixed_gqa_attention(layers[0].q, layers[0].kp, layers[0].vp, tokens, c.cu_seqlens, c.kv_lens,
                                    c.slot_ids, c.block_table)
        torch.cuda.synchronize()
        want, written = ref.mixed_attention(case.q, layers[0].kp.cpu(), layers[0].vp.cpu(), case.cu_seqlens,
                                            case.kv_lens, case.slot_ids, case.block_table)
        err = (o[0].float().cpu() - want)[written].abs().max().item()

        def call(i):
            L = layers[i]
            return lambda: cie.mixed_gqa_attention(L.q, L.kp, L.vp, tokens, c.cu_seqlens, c.kv_lens, c.slot_ids,
                                                   c.block_table)
        us, _ = time_calls([call(i) for i in range(R)], args.steps, args.warmup, not args.no_graph, args.repeats)
        us_p, same = time_mixed_planned(cie, layers, c, case, tokens, 14, args)
        pub = PUBLISHED_MIXED_T128[B]
        log(f"feature-bench shape B={B}: {us:.2f} us, planned {us_p:.2f} us (reference, RTX 4070 Laptop: "
            f"{pub} us), err {err:.1e}, planned == unplanned: {same}")
        table.append({"batch": B, "us_per_call": round(us, 2), "us_per_call_planned": round(us_p, 2),
                      "published_us": pub, "speedup_vs_published": round(pub / us, 2),
                      "parity_max_abs_err": err, "planned_equals_unplanned": same})
    b32 = table[-1]
    print(json.dumps({
        "metric": "mixed attention us/call at the reference feature-bench shape (T=128, context 256)",
        "value": b32["us_per_call"], "unit": "us/call", "higher_is_better": False, "n_gpus": 1,
        "vs_published_rtx4070_laptop": b32["speedup_vs_published"], "table": table,
        "dtype": "fp16 (fp32 accumulate)", "data": "synthetic (shuffled pages)",
        "config": {"workload": "B sequences share 128 new tokens on 256 cached tokens each, one layer",
                   "tokens": tokens, "context": context, "max_seqlen": tokens},
    }), flush=True)


def bench_model(args, cie, dev, n_requests: int = 64, n_slots: int = 33, new_tokens: int = 128,
                budget: int = 512, sigma: float = 0.5):
    """Config 5: a 24-layer Qwen2.5-0.5B-shaped model (random fp16 weights) served end to end.

    Continuous batching (``Scheduler``, the reference's policy): `n_requests`
    prompts (lognormal lengths, median 256, sigma recorded, clipped to
    [16, 2048]) through `n_slots - 1` slots, a token budget of `budget` per
    step and a 32,768-token pool; each request generates `new_tokens` tokens
    (no EOS: random weights).  Prefill chunks and decode rows are packed into
    eager mixed steps; pure decode steps replay the hipGraph of the batch
    bucket (every layer: one rope + append + split-KV decode launch).
    Reported: output tokens/s over the whole run (the metric), steps,
    preemptions; then, on 32 resident sequences, the steady-state decode step,
    its graph replay alone and the attention launches of one step alone.
    """
    from transformers import Qwen2Config, Qwen2ForCausalLM
    from custom_inference_engine_amd.scheduler import Scheduler, assign_pages

    cfg = Qwen2Config(hidden_size=896, num_attention_heads=14, num_key_value_heads=2, intermediate_size=4864,
                      num_hidden_layers=24, vocab_size=151936, max_position_embeddings=32768, rope_theta=1e6,
                      rms_norm_eps=1e-6, tie_word_embeddings=True)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    with torch.device(dev):
        model = Qwen2ForCausalLM(cfg)
    model = model.half().eval()
    cie.use_triton_attention(model)
    kv = cie.KVStorage(cfg, max_cache_len=32768, page_size=16, n_slots=n_slots, device=dev,
                       dtype=torch.float16)
    log(f"config 5: 24 layers, {n_requests} requests, {n_slots - 1} slots, pool {kv.n_pages} pages; "
        f"capturing the decode graphs")
    t0 = time.perf_counter()
    sched = Scheduler(model, kv, eos_token_ids={cfg.vocab_size}, max_new_tokens=new_tokens,
                      token_budget=budget)
    init_s = time.perf_counter() - t0

    # time every step as the loop sees it (each ends in a host sync: .tolist())
    ex = sched.executor
    step_time = {"decode": [], "mixed": []}

    def timed(kind, fn):
        def run(*a):
            t = time.perf_counter()
            out = fn(*a)
            step_time[kind].append((len(a[-1]), time.perf_counter() - t))
            return out
        return run
    ex.decode, ex.mixed = timed("decode", ex.decode), timed("mixed", ex.mixed)

    g = torch.Generator().manual_seed(5)
    lens = torch.exp(torch.randn(n_requests, generator=g) * sigma + math.log(256)).round().clamp(16, 2048).long()
    prompts = [torch.randint(0, cfg.vocab_size, (int(n),), generator=g).tolist() for n in lens]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.inference_mode():
        results = sched.generate(prompts)
    torch.cuda.synchronize()
    run_s = time.perf_counter() - t0
    n_out = sum(len(r.new_tokens) for r in results)
    n_prompt = int(lens.sum())
    st = sched.stats
    dec32 = [dt for n, dt in step_time["decode"] if n == n_slots - 1]
    ttft = sorted(r.t_first - r.t_arrival for r in results)
    log(f"served {n_requests} requests: {n_prompt} prompt + {n_out} output tokens in {run_s:.2f} s; "
        f"{sum(st.decode_steps.values())} decode + {sum(st.mixed_steps.values())} mixed steps, "
        f"{st.preemptions} preemptions")

    # steady state on 32 resident sequences (the bucket-32 graph of the same executor)
    batch = n_slots - 1
    dec = ex.decode_module(batch)
    slots = list(range(1, batch + 1))
    free = (torch.randperm(kv.n_pages - 1, generator=g) + 1).tolist()
    extra = 64
    for sl, p in zip(slots, prompts[:batch]):
        assign_pages(kv, sl, len(p) + new_tokens + extra, free)
    with torch.inference_mode():
        done = [0] * batch
        while any(d < len(p) for d, p in zip(done, prompts)):
            chunk, chunk_slots, left = [], [], budget
            for i, p in enumerate(prompts[:batch]):
                if done[i] < len(p) and left > 0:
                    n = min(len(p) - done[i], left)
                    chunk.append(p[done[i]:done[i] + n])
                    chunk_slots.append(slots[i])
                    done[i] += n
                    left -= n
            if not chunk:
                break
            ex.mixed_module(sum(map(len, chunk))).forward(chunk, chunk_slots)
        for _ in range(3):
            dec.forward(slots)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(new_tokens - 3):
            dec.forward(slots)
        torch.cuda.synchronize()
        step_us = (time.perf_counter() - t0) / (new_tokens - 3) * 1e6
        n_rep = extra - 8
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(n_rep):
            dec.step.replay()
        end.record()
        torch.cuda.synchronize()
        replay_us = start.elapsed_time(end) * 1e3 / n_rep
        # the attention launches of one step alone: 24 one-launch rope + append + decode calls
        qkv = torch.randn(1, batch, (14 + 4) * 64, device=dev, dtype=torch.float16)
        cos = torch.ones(1, batch, 64, device=dev, dtype=torch.float16)
        sin = torch.zeros(1, batch, 64, device=dev, dtype=torch.float16)
        slot_t = torch.tensor(slots, device=dev)

        def attn_step():
            for layer in range(cfg.num_hidden_layers):
                cie.decode_qkv_rope_gqa_attention(qkv, cos, sin, kv.keys[layer], kv.values[layer], kv.lens,
                                                  slot_t, kv.block_table, num_heads=14)
        attn_us, _ = time_calls([attn_step], 40, 8, True, 3)
    ctx = float((kv.lens[slots].float().mean()).item())
    line = {
        "metric": "config 5 output tokens/s (24-layer Qwen2.5-0.5B shape, continuous batching of 64 requests)",
        "value": round(n_out / run_s, 1), "unit": "tokens/s", "higher_is_better": True,
        "n_gpus": 1, "steps": sum(st.decode_steps.values()) + sum(st.mixed_steps.values()),
        "wall_s": round(run_s, 3), "init_s": round(init_s, 2),
        "total_tokens_per_s": round((n_out + n_prompt) / run_s, 1),
        "decode_steps": sum(st.decode_steps.values()), "mixed_steps": sum(st.mixed_steps.values()),
        "preemptions": st.preemptions, "recomputed_tokens": st.recomputed_tokens,
        "decode_step_ms_at_b32_in_run": round(sorted(dec32)[len(dec32) // 2] * 1e3, 3) if dec32 else None,
        "ttft_ms_median": round(ttft[len(ttft) // 2] * 1e3, 1),
        "steady_state_b32": {"decode_step_us": round(step_us, 1), "tokens_per_s": round(batch / (step_us * 1e-6), 1),
                             "graph_replay_us": round(replay_us, 1), "attention_us_per_step": round(attn_us, 1),
                             "attention_share_of_replay": round(attn_us / replay_us, 3),
                             "mean_context": round(ctx, 1)},
        "dtype": "fp16 (fp32 accumulate)", "data": "synthetic (random weights, random prompt ids)",
        "config": {"workload": "Qwen2.5-0.5B-shaped forward, random init from a local Qwen2Config, "
                               "reference scheduling policy",
                   "layers": 24, "requests": n_requests, "slots": n_slots - 1, "prompt_len_median": 256,
                   "prompt_len_sigma": sigma, "prompt_tokens": n_prompt, "new_tokens": new_tokens,
                   "token_budget": budget, "pool_tokens": 32768},
    }
    print(json.dumps(line), flush=True)


def bench_step_modules(args, cie, dev, n_seqs: int = 8, new_tokens: int = 64, prior: int = 512,
                       bucket: int = 512, steps: int = 20, warmup: int = 3):
    """One mixed step of config 5's 24-layer model through each step module.

    8 sequences of 64 new tokens over 512 cached ones in the 512-token bucket
    (`MixedModule` eager, `FullMixedModule` one hipGraph, `PiecewiseMixedModule`
    graph pieces between eager attention calls).  A step = host upload + the
    step, ended by a device sync; the cached lengths are set back to `prior`
    before each step (one small device write, in every mode), so every step
    does the same work.  Random fp16 weights; ms per step, mean of `steps`."""
    from transformers import Qwen2Config, Qwen2ForCausalLM
    from custom_inference_engine_amd.scheduler import (FullMixedModule, MixedModule, PiecewiseMixedModule,
                                                       assign_pages)

    cfg = Qwen2Config(hidden_size=896, num_attention_heads=14, num_key_value_heads=2, intermediate_size=4864,
                      num_hidden_layers=24, vocab_size=151936, max_position_embeddings=32768, rope_theta=1e6,
                      rms_norm_eps=1e-6, tie_word_embeddings=True)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    with torch.device(dev):
        model = Qwen2ForCausalLM(cfg)
    model = model.half().eval()
    cie.use_triton_attention(model)
    out = {}
    for kind in ("eager", "full_graph", "piecewise"):
        torch._dynamo.reset()
        kv = cie.KVStorage(cfg, max_cache_len=16384, page_size=16, n_slots=33, device=dev, dtype=torch.float16)
        pool = torch.cuda.graph_pool_handle()
        t0 = time.perf_counter()
        if kind == "eager":
            mod = MixedModule(model, kv, token_count=bucket)
        elif kind == "full_graph":
            mod = FullMixedModule(model, kv, batch_size=kv.n_slots - 1, token_count=bucket, pool=pool)
        else:
            buf = torch.zeros((1, bucket, cfg.num_attention_heads, 64), dtype=torch.float16, device=dev)
            mod = PiecewiseMixedModule(model, kv, token_count=bucket, buffer=buf, pool=pool)
        build_s = time.perf_counter() - t0
        free = list(range(1, kv.n_pages))
        slots = list(range(1, n_seqs + 1))
        for sl in slots:
            assign_pages(kv, sl, prior + new_tokens, free)
        slot_t = torch.tensor(slots, device=dev)
        prompts = [[5] * new_tokens for _ in slots]

        def step():
            kv.lens[slot_t] = prior
            mod.upload(prompts, slots)
            return mod.run()

        with torch.inference_mode():
            for _ in range(warmup):
                step()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                step()
            torch.cuda.synchronize()
            ms = (time.perf_counter() - t0) / steps * 1e3
        out[kind] = {"ms_per_step": round(ms, 3), "build_s": round(build_s, 2)}
        log(f"{kind}: {ms:.3f} ms per step (module built in {build_s:.1f} s)")
        del mod, kv
        torch.cuda.empty_cache()
    line = {"metric": "config 5 model: mixed step ms by step module (diagnostic, not a bench line)",
            "unit": "ms/step", "higher_is_better": False, "modules": out,
            "dtype": "fp16 (fp32 accumulate)", "data": "synthetic (random weights, constant token ids)",
            "config": {"workload": "24-layer Qwen2.5-0.5B shape, one mixed step", "sequences": n_seqs,
                       "new_tokens": new_tokens, "cached_tokens": prior, "token_bucket": bucket,
                       "steps": steps}}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
