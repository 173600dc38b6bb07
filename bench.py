#!/usr/bin/env python3
"""Benchmark of ane's quantized compute path on one MI355X.

Headline (BASELINE.json metric, config 2): Op::dense_fused_i8 at
M = N = K = 4096, scale 1.0, ReLU -- fp32 A and B quantized per tensor to
int8, int8 x int8 -> int32 on MFMA, fused dequant/scale/ReLU epilogue.  One
step = one full dense_fused_i8 call with A and B already resident in HBM.
``value`` is 2*M*N*K / (time per step) in TOPS.

Also reported (same JSON line):
* ``roofline`` -- the dominant kernel (the MFMA contraction + epilogue),
  timed alone with HIP events on its stream, against 5.0 POPS int8 dense.
* ``q8_0_matvec`` -- config 3: Q8_0 matvec 14336x4096 ("G mode", x quantized
  on the fly) and the reference-arithmetic opcode 0x57 ("R mode"), GB/s
  against 8 TB/s, rotating >256 MB of weight copies so the Infinity Cache
  cannot serve them.
* ``measured_ceilings`` -- what this GPU sustains (bench_peaks.so, built from
  bench_peaks.hip beside this file):
  an int8 MFMA loop without memory traffic on random operands, with the
  clock it holds, and plain HBM read/write streams; each roofline also
  carries ``frac_measured`` against the matching ceiling.
* ``cpu_baseline`` -- the scalar CPU restatement (oracle/) on a bounded
  sample of the same workload, with the host thread count used.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "int8 GEMM TOPS (% MFMA peak) + q8_0 matvec GB/s (% HBM peak), 1 MI355X"
PEAK_INT8_TOPS = 5000.0   # MI355X dense int8 MFMA, 5.0 POPS
PEAK_HBM_GBS = 8000.0     # MI355X HBM3E, 8 TB/s
PROFILES = ROOT / "profiles"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--M", type=int, default=4096)
    ap.add_argument("--N", type=int, default=4096)
    ap.add_argument("--K", type=int, default=4096)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-q8", action="store_true", help="skip the Q8_0 matvec / mul_mat sections")
    ap.add_argument("--no-sweep", action="store_true", help="skip the dense_fused_i8 M sweep")
    ap.add_argument("--no-decode", action="store_true", help="skip the config-5 decode step")
    ap.add_argument("--layers", type=int, default=32, help="decoder layers of the config-5 model")
    ap.add_argument("--kernel-reps", type=int, default=200, help="launches per kernel timing")
    ap.add_argument("--eager", action="store_true",
                    help="launch every step from Python instead of replaying the steps as one HIP graph")
    ap.add_argument("--only", choices=["gemm", "fused", "q8g", "q8r", "copy", "decode", "qformats", "ceilings",
                             "mulmat", "msweep", "mnist", "mfma_loop", "vendor_int8", "igemm", "rotating"],
                    default=None,
                    help="profiling mode: launch only this workload --steps times, print timing")
    return ap.parse_args()


WARM_S = 0.25  # seconds of warm-up replays before a timed region (the clock settles within ~20 ms)


def warm_until(replay, stream, min_s: float = WARM_S) -> int:
    """Call replay() (enqueueing GPU work on ``stream``) back to back until
    at least min_s seconds have passed, at least once; returns the count."""
    t0 = time.perf_counter()
    n = 0
    while n == 0 or time.perf_counter() - t0 < min_s:
        replay()
        n += 1
        if n % 8 == 0:
            stream.synchronize()  # keep the host within a few replays of the GPU
    stream.synchronize()
    return n


def events_time(fn, reps: int, stream) -> float:
    """Average milliseconds per call of fn() over reps calls, HIP events on stream."""
    import torch

    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(reps):
        fn()
    stop.record(stream)
    stop.synchronize()
    return start.elapsed_time(stop) / reps


def graph_time(fn_s, reps: int, rounds: int = 5) -> float:
    """Median milliseconds per call of fn_s(stream): `reps` calls (fn_s may
    rotate its inputs) are captured into one HIP graph on a side stream,
    replayed back to back for 0.1 s to warm up, then replayed `rounds` times
    on that stream between HIP events, so host launch overhead is outside
    the timed region."""
    import torch

    gs = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(gs):
        for _ in range(3):
            fn_s(gs)
        gs.synchronize()
        with torch.cuda.graph(graph, stream=gs):
            for _ in range(reps):
                fn_s(gs)
        warm_until(graph.replay, gs, 0.1)
        times = []
        for _ in range(rounds):
            start = torch.cuda.Event(enable_timing=True)
            stop = torch.cuda.Event(enable_timing=True)
            start.record(gs)
            graph.replay()
            stop.record(gs)
            stop.synchronize()
            times.append(start.elapsed_time(stop) / reps)
    times.sort()
    return times[len(times) // 2]


def read_pmc_traffic(name: str):
    """HBM bytes per launch from a committed rocprofv3 --pmc summary
    (profiles/<name>), lines 'traffic_bytes_per_launch: <int>'."""
    p = PROFILES / name
    if not p.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", p.read_text())
    return float(m.group(1)) if m else None


def read_profile_value(name: str, key: str):
    """A 'key: <number>' line of a committed profile summary (profiles/<name>)."""
    p = PROFILES / name
    if not p.exists():
        return None
    m = re.search(rf"^{re.escape(key)}:\s*([0-9.eE+]+)", p.read_text(), flags=re.M)
    return float(m.group(1)) if m else None


def main() -> int:
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build targets one GPU: the dense_fused_i8 and Q8_0 "
                                   "kernels shard by rows with no reduction; "
                                   "run with --gpus 1"}), flush=True)
        return 2

    import numpy as np
    import torch

    import ane_amd

    ane_amd.require_gpu()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    M, N, K = args.M, args.N, args.K

    # ------------------------------------------------------------ inputs
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    A = torch.randn((M, K), generator=g, device=dev, dtype=torch.float32)
    B = torch.randn((K, N), generator=g, device=dev, dtype=torch.float32)
    C = torch.empty((M, N), device=dev, dtype=torch.float32)
    wsb = ane_amd.dense_fused_i8_workspace_size(M, N, K)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    scales = torch.empty(2, dtype=torch.float32, device=dev)

    # the wait record of the quantizer is checked once after each timed
    # section (ane_amd.dense_fused_i8_status), not after every call
    def fused(st=stream):
        ane_amd.dense_fused_i8(M, N, K, 1.0, True, A, B, C, workspace=ws, stream=st, check_wait=False)

    def gemm_phase(st=stream):
        ane_amd.dense_fused_i8_gemm(M, N, K, 1.0, True, C, ws, stream=st)

    def quant_phase(st=stream):
        ane_amd.dense_fused_i8_quantize(M, N, K, A, B, ws, stream=st, check_wait=False)

    ops = 2.0 * M * N * K

    if args.only == "copy":
        # Plain device copy of a known size: the reference reading for the
        # FETCH_SIZE / WRITE_SIZE scale factors of the --pmc runs.
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.warmup):
            dst.copy_(src)
        ms = events_time(lambda: dst.copy_(src), args.steps, stream)
        log(f"copy 256 MiB: {ms * 1e3:.2f} us/launch, {2 * (256 << 20) / ms / 1e6:.0f} GB/s")
        return 0
    if args.only in ("q8g", "q8r"):
        return profile_q8(args, stream)
    if args.only == "msweep":
        print(json.dumps(bench_m_sweep(args, N, K)), flush=True)
        return 0
    if args.only == "mnist":
        print(json.dumps(bench_mnist(args)), flush=True)
        return 0
    if args.only == "igemm":
        print(json.dumps(bench_igemm(args)), flush=True)
        return 0
    if args.only == "rotating":
        print(json.dumps(headline_rotating(args, M, N, K, ops)), flush=True)
        return 0
    if args.only == "mulmat":
        print(json.dumps(bench_mul_mat(args)), flush=True)
        return 0
    if args.only == "ceilings":
        print(json.dumps(measured_ceilings(args)), flush=True)
        return 0
    if args.only == "qformats":
        bench_qformats(args)
        return 0
    if args.only == "decode":
        bench_decode(args)
        return 0

    if args.only == "vendor_int8":
        # a vendor comparison point, not part of the product: torch._int_mm
        # (hipBLASLt on ROCm) on int8 operands of the same shape, int32 out,
        # HIP-graph replayed like the contraction
        a8 = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=dev)
        b8 = torch.randint(-127, 128, (K, N), dtype=torch.int8, device=dev)
        out = torch.empty((M, N), dtype=torch.int32, device=dev)

        def vend(st):
            torch._int_mm(a8, b8, out=out)

        ms = graph_time(vend, args.steps)
        log(f"torch._int_mm int8 {M}x{N}x{K}: {ms * 1e3:.2f} us/launch, {ops / ms / 1e9:.1f} TOPS")
        print(json.dumps({"only": "vendor_int8", "us_per_launch": round(ms * 1e3, 3),
                          "TOPS": round(ops / ms / 1e9, 2)}), flush=True)
        return 0
    if args.only == "mfma_loop":
        # the int8 MFMA loop of bench_peaks.so alone (counter calibration)
        print(json.dumps(mfma_loop_only(args)), flush=True)
        return 0
    if args.only in ("gemm", "fused"):
        # the same HIP-graph replay the headline roofline measures, so a
        # kernel trace of this command reproduces the line's avg_launch_us
        fn = gemm_phase if args.only == "gemm" else fused
        quant_phase()
        torch.cuda.synchronize()
        if args.eager:
            for _ in range(args.warmup):
                fn()
            ms = events_time(fn, args.steps, stream)
        else:
            ms = graph_time(fn, args.steps)
        log(f"{args.only}: {ms * 1e3:.2f} us/launch, {ops / ms / 1e9:.1f} TOPS "
            f"({'eager launches' if args.eager else 'HIP-graph replay, median of 5 rounds'})")
        print(json.dumps({"only": args.only, "us_per_launch": round(ms * 1e3, 3),
                          "TOPS": round(ops / ms / 1e9, 2)}), flush=True)
        return 0

    # ------------------------------------------------------------ headline
    # The K timed steps are K full dense_fused_i8 calls (both quantize passes
    # and the contraction, on fresh fp32 operands each time), captured once
    # into a HIP graph.  The warmup replays a graph of W steps back to back
    # until at least WARM_S seconds have passed, then the timed graph once,
    # untimed (a graph's first replay carries one-time setup): the GPU's
    # clock settles over the first ~20 ms of this workload (measured: a
    # 20-step replay right after start 104 us/step, falling to 95 us/step
    # over ten replays; after 0.3 s of warm replays, 95 us/step at once).
    # The timed replay is bracketed by synchronisations, and its time is
    # read from HIP events recorded on the replay stream just before and
    # after it: all K steps of GPU work, without the host's launch and
    # synchronisation latency (the wall clock around the same replay is
    # reported too).  --eager launches the K calls from Python instead,
    # between the same two events.
    log(f"dense_fused_i8 M={M} N={N} K={K}: warmup {args.warmup}, steps {args.steps}"
        f"{' (eager launches)' if args.eager else ' (one HIP graph of the steps)'}")
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    if args.eager:
        warm_until(lambda: [fused() for _ in range(max(1, args.warmup))], stream)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0.record(stream)
        for _ in range(args.steps):
            fused()
        ev1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    else:
        gs = torch.cuda.Stream()
        warm, timed = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
        with torch.cuda.stream(gs):
            fused(gs)
            gs.synchronize()
            with torch.cuda.graph(warm, stream=gs):
                for _ in range(max(1, args.warmup)):
                    fused(gs)
            with torch.cuda.graph(timed, stream=gs):
                for _ in range(args.steps):
                    fused(gs)
            warm_until(warm.replay, gs)
            timed.replay()
            gs.synchronize()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            ev0.record(gs)
            timed.replay()
            ev1.record(gs)
            gs.synchronize()
            torch.cuda.synchronize()
            wall = time.perf_counter() - t0
    ane_amd.dense_fused_i8_status(ws)  # every quantize of the timed steps met its grid-wide wait
    ms_per_step = ev0.elapsed_time(ev1) / args.steps
    wall_ms_per_step = wall * 1e3 / args.steps
    value = ops / (ms_per_step * 1e-3) / 1e12
    log(f"whole op: {ms_per_step * 1e3:.2f} us/step = {value:.1f} TOPS "
        f"(wall clock around the replay: {wall_ms_per_step * 1e3:.2f} us/step)")
    rotating = headline_rotating(args, M, N, K, ops)

    # ------------------------------------------------------------ kernel roofline
    # The contraction's launch duration: kernel_reps launches captured into
    # one HIP graph and replayed between HIP events (graph_time).  Its
    # rocprofv3 traces: bench.py --only gemm (the same replay) and --only
    # fused (inside the op).  A second reading brackets each contraction
    # inside eager dense_fused_i8 calls with HIP events; those event packets
    # add their own dispatch latency, so it reads a few us above the kernel.
    quant_phase()
    torch.cuda.synchronize()
    reps = max(20, args.kernel_reps // 4)
    marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for e0, e1 in [(None, None)] * 3 + marks:
        quant_phase()
        if e0 is not None:
            e0.record(stream)
        gemm_phase()
        if e1 is not None:
            e1.record(stream)
    torch.cuda.synchronize()
    ane_amd.dense_fused_i8_status(ws)
    in_op = sorted(e0.elapsed_time(e1) for e0, e1 in marks)
    in_op_ms = sum(in_op) / len(in_op)
    gemm_ms = graph_time(gemm_phase, args.kernel_reps)
    gemm_tops = ops / (gemm_ms * 1e-3) / 1e12
    quant_ms = graph_time(quant_phase, max(20, args.kernel_reps // 4))
    quant_bytes = 5.0 * (M * K + K * N)  # read fp32 once + write int8 (algorithmic)
    log(f"MFMA kernel: {gemm_ms * 1e3:.2f} us = {gemm_tops:.1f} TOPS ({gemm_tops / PEAK_INT8_TOPS:.1%})")
    log(f"quantize phase: {quant_ms * 1e3:.2f} us = {quant_bytes / quant_ms / 1e6:.0f} GB/s algorithmic")
    roofline = {
        "bound": "mfma",
        "kernel": "k_gemm_tile256 (dense_fused_i8 contraction + fused dequant/scale/ReLU epilogue)",
        "achieved": round(gemm_tops, 2),
        "peak": PEAK_INT8_TOPS,
        "unit": "TOPS",
        "frac": round(gemm_tops / PEAK_INT8_TOPS, 4),
        "algorithmic_per_launch": f"2*M*N*K = {int(ops)} int8 ops",
        "avg_launch_us": round(gemm_ms * 1e3, 3),
        "avg_launch_how": (f"{args.kernel_reps} contraction launches as one HIP graph, replayed between HIP "
                           "events (median of 5 replays); rocprofv3 traces: bench.py --only gemm "
                           "(profiles/gemm_i8_tile256_4096_kernel_trace.txt) and, inside the op, --only fused "
                           "(profiles/dense_fused_i8_4096_kernel_trace.txt)"),
        "in_op_events_us": round(in_op_ms * 1e3, 3),
        "in_op_events_how": (f"HIP events around the contraction inside {reps} eager dense_fused_i8 calls on one "
                             "stream (mean); includes the event packets' dispatch latency"),
        "traffic": read_pmc_traffic("gemm_i8_4096_pmc.txt"),
        "mfma_util": read_profile_value("gemm_i8_4096_mfma_pmc.txt", "mfma_util"),
        "held_clock_GHz": read_profile_value("gemm_i8_4096_mfma_pmc.txt", "held_clock_GHz"),
        "mfma_util_how": ("SQ_VALU_MFMA_BUSY_CYCLES per SIMD / SQ_BUSY_CYCLES per SE over the contraction's "
                          "dispatch (rocprofv3 --pmc, profiles/gemm_i8_4096_mfma_pmc.txt); the clock it held "
                          "is SQ_BUSY_CYCLES per SE / dispatch time"),
        "profiles": ["profiles/gemm_i8_tile256_4096_kernel_trace.txt",
                     "profiles/dense_fused_i8_4096_kernel_trace.txt", "profiles/gemm_i8_4096_pmc.txt",
                     "profiles/gemm_i8_4096_mfma_pmc.txt", "profiles/gemm_i8_4096_lds_pmc.txt"],
    }
    if roofline["held_clock_GHz"]:
        # the same kernel against the peak at the clock it holds (8192 int8 ops/clk/CU)
        held_peak = 8192 * torch.cuda.get_device_properties(0).multi_processor_count * roofline["held_clock_GHz"] / 1e3
        roofline["frac_at_held_clock"] = round(gemm_tops / held_peak, 4)

    ceilings = measured_ceilings(args)
    mfma_meas = ceilings["mfma_i8_loop_workload"]["TOPS"]
    roofline["measured_peak"] = mfma_meas
    roofline["frac_measured"] = round(gemm_tops / mfma_meas, 4)
    roofline["measured_peak_how"] = ("int8 MFMA loop with no memory traffic on operands drawn like the workload's "
                                     "(N(0,1) quantized by absmax; clock "
                                     f"{ceilings['mfma_i8_loop_workload']['clock_GHz']} GHz)")

    # ------------------------------------------------------------ Q8_0 matvec
    q8 = None
    mul_mat = None
    if not args.no_q8:
        q8 = bench_q8(args, stream)
        rd = ceilings["hbm_read_62MB"]["GB_s"]
        q8["roofline"]["measured_peak"] = rd
        q8["roofline"]["frac_measured"] = round(q8["roofline"]["achieved"] / rd, 4)
        q8["roofline"]["measured_peak_how"] = "plain read of the same 62 MB, rotating buffers"
        mul_mat = bench_mul_mat(args)
    qformats = bench_qformats(args) if not args.no_q8 else None
    m_sweep = bench_m_sweep(args, N, K) if not args.no_sweep else None
    mnist = bench_mnist(args) if not args.no_sweep else None
    igemm = bench_igemm(args) if not args.no_sweep else None
    decode = bench_decode(args) if not args.no_decode else None

    # ------------------------------------------------------------ CPU baseline
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(A, B, C, M, N, K)

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: A, B ~ N(0,1) fp32 (seeded), quantized per tensor on the GPU each step",
        "timing": ("eager launches from Python between HIP events" if args.eager else
                   "the K steps captured as one HIP graph, replayed once untimed after the warmup and "
                   "then once between synchronisations; ms_per_step from HIP events recorded on the "
                   "replay stream around that replay"),
        "warmup_how": (f"the W warmup steps (one HIP graph) replayed back to back for at least {WARM_S} s, "
                       "so the GPU's clock has settled before the K timed steps"),
        "wall_ms_per_step": round(wall_ms_per_step, 5),
        "rotating_operands": rotating,
        "config": {"workload": f"dense_fused_i8 M={M} N={N} K={K} scale=1.0 relu (config 2)",
                   "M": M, "N": N, "K": K},
        "roofline": roofline,
        "phases_us": {"quantize": round(quant_ms * 1e3, 2), "contraction": round(gemm_ms * 1e3, 2)},
        "measured_ceilings": ceilings,
        "q8_0_matvec": q8,
        "q8_0_mul_mat_config4": mul_mat,
        "other_formats_gemv": qformats,
        "dense_fused_m_sweep": m_sweep,
        "mnist_mlp_config1": mnist,
        "cblas_igemm_1024": igemm,
        "decode_config5": decode,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


def headline_rotating(args, M, N, K, ops) -> dict:
    """The headline step again with the operands rotating over three A/B
    sets (3 x 128 MiB of fp32 at 4096^3, more than the 256 MB Infinity
    Cache), each set with its own output and workspace, so the quantize
    phase reads operands that the previous steps did not leave in the
    cache.  Same graph capture and HIP-event timing as the headline."""
    import torch

    import ane_amd

    dev = torch.device("cuda:0")
    nsets = 3
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    wsb = ane_amd.dense_fused_i8_workspace_size(M, N, K)
    sets = [(torch.randn((M, K), generator=g, device=dev), torch.randn((K, N), generator=g, device=dev),
             torch.empty((M, N), device=dev), torch.empty(wsb, dtype=torch.uint8, device=dev))
            for _ in range(nsets)]
    steps = max(args.steps, nsets)
    steps -= steps % nsets
    gs = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(gs):
        for A, B, C, ws in sets:
            ane_amd.dense_fused_i8(M, N, K, 1.0, True, A, B, C, workspace=ws, stream=gs, check_wait=False)
        gs.synchronize()
        with torch.cuda.graph(graph, stream=gs):
            for i in range(steps):
                A, B, C, ws = sets[i % nsets]
                ane_amd.dense_fused_i8(M, N, K, 1.0, True, A, B, C, workspace=ws, stream=gs, check_wait=False)
        warm_until(graph.replay, gs)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(gs)
        graph.replay()
        e1.record(gs)
        gs.synchronize()
    for *_, ws in sets:
        ane_amd.dense_fused_i8_status(ws)
    ms = e0.elapsed_time(e1) / steps
    log(f"whole op, operands rotating over {nsets} sets: {ms * 1e3:.2f} us/step = {ops / ms / 1e9:.1f} TOPS")
    res = {"us_per_step": round(ms * 1e3, 3), "TOPS": round(ops / ms / 1e9, 2), "sets": nsets,
           "steps": steps, "operand_bytes_per_set": 4 * (M * K + K * N),
           "how": ("A, B (fp32), C and the workspace rotate over 3 sets, step i using set i % 3, one HIP "
                   "graph replayed between HIP events")}
    del sets, graph
    torch.cuda.empty_cache()
    return res


def profile_q8(args, stream) -> int:
    """Launch only the 14336x4096 Q8_0 matvec (G or R mode) --steps times."""
    import numpy as np
    import torch

    import ane_amd
    from tests import data

    Nr, Kc = 14336, 4096
    W0 = torch.from_numpy(data.q8_0_weights(Nr, Kc, seed=3)).cuda()
    copies = 6
    Ws = [W0] + [W0.clone() for _ in range(copies - 1)]
    x = torch.from_numpy(data.activations(1, Kc, seed=4)).cuda()
    y = torch.empty(Nr, device="cuda", dtype=torch.float32)
    wsq = torch.empty(ane_amd.q8_0_mul_mat_workspace_size(Kc, 1), dtype=torch.uint8, device="cuda")
    it = [0]

    def fn():
        W = Ws[it[0] % copies]
        it[0] += 1
        if args.only == "q8g":
            ane_amd.q8_0_mul_mat(Nr, Kc, 1, x, W, y, workspace=wsq, stream=stream)
        else:
            ane_amd.q8_0_gemv(Nr, Kc, x, W, y, stream=stream)

    for _ in range(args.warmup):
        fn()
    ms = events_time(fn, args.steps, stream)
    alg = Nr * (Kc // 32) * 34 + 4 * Kc + 4 * Nr
    log(f"{args.only} {Nr}x{Kc}: {ms * 1e3:.2f} us/launch, {alg / ms / 1e6:.0f} GB/s")
    return 0


def _peaks():
    import ctypes

    peaks = ctypes.CDLL(str(ROOT / "bench_peaks.so"))
    u32, u64, vp, i32 = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_int
    peaks.ane_peak_mfma_i8.argtypes = [u32, u32, u32, vp, vp, vp, vp]
    peaks.ane_peak_read.argtypes = [vp, u64, u32, i32, vp, vp]
    peaks.ane_peak_write.argtypes = [vp, u64, u32, vp]
    return peaks


def mfma_loop_only(args) -> dict:
    """The int8 MFMA loop on workload-distributed operands, --steps launches:
    the reference kernel for reading MFMA counters (its ops, time and
    in-kernel clock are known)."""
    import ctypes

    import torch

    peaks = _peaks()
    dev = torch.device("cuda:0")
    ncu = torch.cuda.get_device_properties(0).multi_processor_count
    st = torch.cuda.current_stream()
    wgs, threads, iters = ncu, 512, 16000
    sums = torch.empty(wgs * threads, dtype=torch.int32, device=dev)
    clocks = torch.zeros(4, dtype=torch.int64, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    gauss = torch.randn(16384, generator=g, device=dev)
    data = torch.round(gauss * (127.0 / gauss.abs().max())).to(torch.int8)
    ops = wgs * (threads // 64) * iters * 8 * 65536
    fn = lambda: peaks.ane_peak_mfma_i8(wgs, threads, iters, data.data_ptr(), sums.data_ptr(), clocks.data_ptr(),
                                        ctypes.c_void_p(st.cuda_stream))
    fn()
    ms = events_time(fn, args.steps, st)
    c = clocks.cpu().tolist()
    ghz = (c[1] - c[0]) / ((c[3] - c[2]) / 100e6) / 1e9
    tops = ops / (ms * 1e-3) / 1e12
    log(f"MFMA loop (workload operands): {ms * 1e3:.2f} us/launch, {tops:.0f} TOPS at {ghz:.3f} GHz")
    return {"only": "mfma_loop", "us_per_launch": round(ms * 1e3, 3), "TOPS": round(tops, 1),
            "clock_GHz": round(ghz, 3), "ops_per_launch": ops}


def measured_ceilings(args) -> dict:
    """Ceilings measured on this GPU with bench_peaks.so, reported
    beside the datasheet peaks: an int8 MFMA loop with no memory traffic on
    random operands (the clock the chip holds under it, from s_memtime over
    s_memrealtime) and on constant operands, and plain HBM read / write
    streams at the sizes the roofline kernels move."""
    import ctypes

    import torch

    peaks = _peaks()
    dev = torch.device("cuda:0")
    ncu = torch.cuda.get_device_properties(0).multi_processor_count
    st = torch.cuda.current_stream()
    sp = ctypes.c_void_p(st.cuda_stream)

    def check(rc):
        if rc != 0:
            raise RuntimeError("bench_peaks launch failed")

    out = {"cus": ncu}
    wgs, threads, iters = ncu, 512, 16000
    sums = torch.empty(wgs * threads, dtype=torch.int32, device=dev)
    clocks = torch.zeros(4, dtype=torch.int64, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    gauss = torch.randn(16384, generator=g, device=dev)
    gauss = torch.round(gauss * (127.0 / gauss.abs().max())).to(torch.int8)  # the workload's operand distribution
    operands = {"random": torch.randint(-128, 128, (16384,), generator=g, dtype=torch.int8, device=dev),
                "workload": gauss,
                "constant": torch.ones(16384, dtype=torch.int8, device=dev)}
    ops = wgs * (threads // 64) * iters * 8 * 65536
    for kind, data in operands.items():
        fn = lambda: check(peaks.ane_peak_mfma_i8(wgs, threads, iters, data.data_ptr(), sums.data_ptr(),
                                                  clocks.data_ptr(), sp))
        fn()
        ms = events_time(fn, 10, st)
        c = clocks.cpu().tolist()
        ghz = (c[1] - c[0]) / ((c[3] - c[2]) / 100e6) / 1e9
        tops = ops / (ms * 1e-3) / 1e12
        out[f"mfma_i8_loop_{kind}"] = {"TOPS": round(tops, 1), "clock_GHz": round(ghz, 3),
                                       "frac_datasheet": round(tops / PEAK_INT8_TOPS, 4)}
        log(f"MFMA loop, {kind} operands: {tops:.0f} TOPS ({tops / PEAK_INT8_TOPS:.1%}) at {ghz:.2f} GHz")
    out["mfma_i8_loop_how"] = (f"{wgs} workgroups x 8 waves, 8 independent v_mfma_i32_32x32x32_i8 chains "
                               "per wave, operands cycled through 8 A and 8 B fragments, no memory traffic")
    del sums

    hit = torch.zeros(1, dtype=torch.int32, device=dev)

    def read_rate(nbytes, nbuf, reps):
        """Best of 2, 4 and 8 workgroups per CU: (GB/s, us, workgroups per CU)."""
        bufs = [torch.ones(nbytes, dtype=torch.uint8, device=dev) for _ in range(nbuf)]
        best = None
        for wpc in (2, 4, 8):
            k = [0]

            def rd(s):
                check(peaks.ane_peak_read(bufs[k[0] % nbuf].data_ptr(), nbytes, wpc * ncu, 12345, hit.data_ptr(),
                                          ctypes.c_void_p(s.cuda_stream)))
                k[0] += 1

            ms = graph_time(rd, reps)
            if best is None or ms < best[1]:
                best = (nbytes / ms / 1e6, ms, wpc)
        del bufs
        torch.cuda.empty_cache()
        return best

    nb = 62_390_272  # the 14336x4096 Q8_0 matrix
    gbs, ms, wpc = read_rate(nb, 6, 24)
    out["hbm_read_62MB"] = {"GB_s": round(gbs, 1), "us": round(ms * 1e3, 3),
                            "how": "16-byte non-temporal loads, each workgroup a contiguous range, "
                                   f"{wpc} workgroups per CU (best of 2/4/8), 6 rotating 62,390,272-byte "
                                   "buffers (> Infinity Cache)"}
    log(f"HBM read 62 MB: {ms * 1e3:.2f} us = {gbs:.0f} GB/s")
    gbs, ms, wpc = read_rate(1 << 30, 2, 4)
    out["hbm_read_1GiB"] = {"GB_s": round(gbs, 1), "us": round(ms * 1e3, 3),
                            "how": f"as hbm_read_62MB over 2 rotating 1 GiB buffers ({wpc} workgroups per CU): "
                                   "the rate without the launch ramp"}
    log(f"HBM read 1 GiB: {ms * 1e3:.2f} us = {gbs:.0f} GB/s")
    wb = 64 << 20
    wbufs = [torch.empty(wb, dtype=torch.uint8, device=dev) for _ in range(5)]
    best = None
    for wpc in (2, 4, 8):
        def wr(s, wpc=wpc):
            check(peaks.ane_peak_write(wbufs[k[0] % 5].data_ptr(), wb, wpc * ncu, ctypes.c_void_p(s.cuda_stream)))
            k[0] += 1

        k = [0]
        ms = graph_time(wr, 20)
        if best is None or ms < best[0]:
            best = (ms, wpc)
    ms, wpc = best
    out["hbm_write_64MiB"] = {"GB_s": round(wb / ms / 1e6, 1), "us": round(ms * 1e3, 3),
                              "how": f"16-byte non-temporal stores, contiguous per workgroup, {wpc} workgroups "
                                     "per CU (best of 2/4/8), 5 rotating 64 MiB buffers"}
    log(f"HBM write 64 MiB: {ms * 1e3:.2f} us = {wb / ms / 1e6:.0f} GB/s")
    del wbufs
    torch.cuda.empty_cache()
    return out


def bench_q8(args, stream) -> dict:
    import numpy as np
    import torch

    import ane_amd
    from tests import data

    res = {}
    shapes = [(14336, 4096), (4096, 4096), (4096, 14336)]
    for (Nr, Kc) in shapes:
        row_bytes = Kc // 32 * 34
        wbytes = Nr * row_bytes
        copies = max(2, int(np.ceil(300e6 / wbytes)))  # > 256 MB Infinity Cache
        W0 = torch.from_numpy(data.q8_0_weights(Nr, Kc, seed=3)).cuda()
        Ws = [W0] + [W0.clone() for _ in range(copies - 1)]
        x = torch.from_numpy(data.activations(1, Kc, seed=4)).cuda()
        y = torch.empty(Nr, device="cuda", dtype=torch.float32)
        wsq = torch.empty(ane_amd.q8_0_mul_mat_workspace_size(Kc, 1), dtype=torch.uint8, device="cuda")
        it = [0]

        def g_mode(st):
            W = Ws[it[0] % copies]
            it[0] += 1
            ane_amd.q8_0_mul_mat(Nr, Kc, 1, x, W, y, workspace=wsq, stream=st)

        def r_mode(st):
            W = Ws[it[0] % copies]
            it[0] += 1
            ane_amd.q8_0_gemv(Nr, Kc, x, W, y, stream=st)

        alg = wbytes + 4 * Kc + 4 * Nr
        entry = {"weights_bytes": wbytes, "algorithmic_bytes": alg, "rotating_copies": copies}
        for name, fn in (("g_mode", g_mode), ("r_mode", r_mode)):
            ms = graph_time(fn, 4 * copies)
            gbs = alg / (ms * 1e-3) / 1e9
            entry[name] = {"us": round(ms * 1e3, 3), "GB_s": round(gbs, 1),
                           "frac_hbm": round(gbs / PEAK_HBM_GBS, 4)}
            log(f"q8_0 {name} {Nr}x{Kc}: {ms * 1e3:.2f} us = {gbs:.0f} GB/s ({gbs / PEAK_HBM_GBS:.1%})")
        res[f"{Nr}x{Kc}"] = entry
        del Ws, W0
        torch.cuda.empty_cache()
    head = res["14336x4096"]["g_mode"]
    return {
        "workload": "Q8_0 matvec 14336x4096, x fp32 quantized to Q8_0 on the fly (G mode), config 3",
        "value": head["GB_s"],
        "unit": "GB/s",
        "roofline": {"bound": "hbm", "achieved": head["GB_s"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": head["frac_hbm"],
                     "algorithmic_per_launch": "N*(K/32)*34 + 4K + 4N bytes",
                     "traffic": read_pmc_traffic("q8_0_matvec_14336x4096_pmc.txt"),
                     "profiles": ["profiles/q8_0_matvec_14336x4096_g_kernel_trace.txt",
                                  "profiles/q8_0_matvec_14336x4096_pmc.txt"]},
        "shapes": res,
    }


def bench_mul_mat(args) -> dict:
    """Config 4: Q8_0 mul_mat (the ggml MUL_MAT hook's kernel, G mode) at the
    Llama-3-8B projections for T = 1, 4, 16, 64 tokens.  GB/s counts the
    weights once plus x and y, as the algorithmic traffic of one call."""
    import numpy as np
    import torch

    import ane_amd
    from tests import data

    res = {}
    for name, (Nr, Kc) in (("qkv", (6144, 4096)), ("o", (4096, 4096)), ("gate_up", (28672, 4096)),
                           ("down", (4096, 14336))):
        wbytes = Nr * (Kc // 32) * 34
        copies = max(2, int(np.ceil(300e6 / wbytes)))
        W0 = torch.from_numpy(data.q8_0_weights(Nr, Kc, seed=5)).cuda()
        Ws = [W0] + [W0.clone() for _ in range(copies - 1)]
        entry = {}
        for T in (1, 4, 16, 64):
            x = torch.from_numpy(data.activations(T, Kc, seed=6)).cuda()
            y = torch.empty(T * Nr, device="cuda", dtype=torch.float32)
            wsq = torch.empty(ane_amd.q8_0_mul_mat_workspace_size(Kc, T, N=Nr), dtype=torch.uint8, device="cuda")
            it = [0]

            def fn(st):
                W = Ws[it[0] % copies]
                it[0] += 1
                ane_amd.q8_0_mul_mat(Nr, Kc, T, x, W, y, workspace=wsq, stream=st)

            ms = graph_time(fn, 2 * copies)
            alg = wbytes + 4 * T * (Kc + Nr)
            entry[f"T{T}"] = {"us": round(ms * 1e3, 2), "GB_s": round(alg / ms / 1e6, 1),
                              "TOPS": round(2.0 * T * Nr * Kc / ms / 1e9, 2)}
            log(f"mul_mat {name} {Nr}x{Kc} T={T}: {ms * 1e3:.2f} us = {alg / ms / 1e6:.0f} GB/s")
        res[f"{name} {Nr}x{Kc}"] = entry
        del Ws, W0
        torch.cuda.empty_cache()
    return {"workload": "config 4: Q8_0 mul_mat G mode, Llama-3-8B projections, T tokens",
            "unit": "us per call", "shapes": res}


def bench_mnist(args) -> dict:
    """Config 1: the MNIST-shaped MLP forward, dense_fused_i8 50x784 -> 128
    (ReLU, scale 1.0) then 128 -> 10 (no ReLU), on the inputs of
    tests/data.py mnist_inputs (80 % exact zeros).  Latency-bound: reported
    as microseconds per forward, through the C entry points in a HIP graph
    and through stream_exec (the opcode boundary, host encoding included).
    Bit-exactness against the oracle is the test
    tests/test_gpu_parity.py::test_dense_fused_mnist_mlp; here the two
    routes are checked against each other."""
    import numpy as np
    import torch

    import ane_amd
    from tests import data

    x, w1, w2 = data.mnist_inputs(seed=1)
    dev = torch.device("cuda:0")
    xd, w1d, w2d = (torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in (x, w1, w2))
    h = torch.zeros(50 * 128, dtype=torch.float32, device=dev)
    o = torch.zeros(50 * 10, dtype=torch.float32, device=dev)
    ws1 = torch.empty(ane_amd.dense_fused_i8_workspace_size(50, 128, 784), dtype=torch.uint8, device=dev)
    ws2 = torch.empty(ane_amd.dense_fused_i8_workspace_size(50, 10, 128), dtype=torch.uint8, device=dev)

    def fwd(st):
        ane_amd.dense_fused_i8(50, 128, 784, 1.0, True, xd, w1d, h, workspace=ws1, stream=st, check_wait=False)
        ane_amd.dense_fused_i8(50, 10, 128, 1.0, False, h, w2d, o, workspace=ws2, stream=st, check_wait=False)

    graph_us = graph_time(fwd, 50) * 1e3
    o_graph = o.clone()
    h2 = torch.zeros_like(h)
    o2 = torch.zeros_like(o)
    recs = [ane_amd.rec_dense_fused_i8(50, 128, 784, 1.0, True, xd, w1d, h2),
            ane_amd.rec_dense_fused_i8(50, 10, 128, 1.0, False, h2, w2d, o2)]
    for _ in range(10):
        ane_amd.stream_exec(recs)
    torch.cuda.synchronize()
    ts = []
    for _ in range(200):
        t0 = time.perf_counter()
        ane_amd.stream_exec(recs)
        torch.cuda.synchronize()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    exec_us = ts[len(ts) // 2] * 1e6
    same = bool(torch.equal(o_graph.view(torch.int32), o2.view(torch.int32)))
    ops = 2 * 50 * 784 * 128 + 2 * 50 * 128 * 10
    log(f"config 1 MLP forward: {graph_us:.2f} us (graph), {exec_us:.1f} us (stream_exec, synchronous)")
    return {"workload": "config 1: dense_fused_i8 50x784->128 ReLU, 128->10, scale 1.0",
            "us_graph": round(graph_us, 2), "us_stream_exec_sync": round(exec_us, 1),
            "ops": ops, "graph_equals_stream_exec": same,
            "parity": "tests/test_gpu_parity.py::test_dense_fused_mnist_mlp (bit-exact against the oracle)"}


def q8_0_random_device(N: int, K: int, gen) -> "torch.Tensor":
    """Q8_0 rows generated on the GPU, distributed as config 3: qs ~ U{-127..127},
    d = fp16(|N(0, 0.01)|).  Returns uint8 [N, K/32*34]."""
    import torch

    nb = K // 32
    W = torch.empty((N, nb, 34), dtype=torch.uint8, device="cuda")
    d = (torch.randn((N, nb), generator=gen, device="cuda") * 0.01).abs().half()
    W[:, :, :2] = d.view(torch.uint8).view(N, nb, 2)
    W[:, :, 2:] = torch.randint(-127, 128, (N, nb, 32), generator=gen, device="cuda",
                                dtype=torch.int8).view(torch.uint8)
    return W.view(N, nb * 34)


def bench_decode(args) -> dict:
    """Config 5: one decode token of a random-init Llama-3-8B-shaped model
    (hidden 4096, FFN 14336, 32 q / 8 kv heads of 128, fp16 KV at context
    4096, Q8_0 weights) through ane_decode_token; every matrix product runs
    on the Q8_0 streaming kernel.  The token is captured once as a HIP graph
    (6 launches per layer) and replayed; mul_mat share = the same graph's
    matrix products alone / the whole token."""
    import ctypes

    import torch

    import ane_amd

    H, F, NH, NKV, HD, CTX = 4096, 14336, 32, 8, 128, 4096
    nl = args.layers
    cfg = ane_amd.DecodeConfig(nl, H, F, NH, NKV, HD, CTX, 1e-5)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    keep = []
    layers = (ane_amd.DecodeLayer * nl)()
    wbytes = 0
    for l in range(nl):
        t = {"w_qkv": q8_0_random_device((NH + 2 * NKV) * HD, H, gen), "w_o": q8_0_random_device(H, NH * HD, gen),
             "w_gate_up": q8_0_random_device(2 * F, H, gen), "w_down": q8_0_random_device(H, F, gen),
             "attn_norm": 1.0 + 0.1 * torch.randn(H, generator=gen, device="cuda"),
             "ffn_norm": 1.0 + 0.1 * torch.randn(H, generator=gen, device="cuda"),
             "k_cache": torch.randn((NKV, CTX, HD), generator=gen, device="cuda").half(),
             "v_cache": torch.randn((NKV, CTX, HD), generator=gen, device="cuda").half()}
        wbytes += sum(t[k].numel() for k in ("w_qkv", "w_o", "w_gate_up", "w_down"))
        keep.append(t)
        layers[l] = ane_amd.DecodeLayer(*[t[k].data_ptr() for k in ("w_qkv", "w_o", "w_gate_up", "w_down",
                                                                      "attn_norm", "ffn_norm", "k_cache",
                                                                      "v_cache")])
    table = torch.from_numpy(ane_amd.rope_table(CTX)).cuda()
    ws = ane_amd.decode_workspace(cfg)
    x = torch.randn(H, generator=gen, device="cuda")
    pos = CTX - 1  # attend over the full 4096-position context
    torch.cuda.synchronize()

    def token(st):
        ane_amd.decode_token(cfg, layers, table, pos, x, ws, stream=st)

    nqkv = (NH + 2 * NKV) * HD
    scratch = torch.empty(2 * F, device="cuda")
    xin = torch.randn(F, generator=gen, device="cuda")

    resid = torch.randn(H, generator=gen, device="cuda")

    # pre-quantized activations for the o and down products (their inputs
    # arrive in the Q8 activation form in the token)
    xq_o = torch.zeros(ane_amd.q8_act_bytes(NH * HD), dtype=torch.uint8, device="cuda")
    xq_d = torch.zeros(ane_amd.q8_act_bytes(F), dtype=torch.uint8, device="cuda")
    xq_g = torch.zeros(ane_amd.q8_act_bytes(F), dtype=torch.uint8, device="cuda")  # the gate|up output
    ane_amd.silu_mul_quant(NH * HD, torch.randn(2 * NH * HD, generator=gen, device="cuda"), xq_o)
    ane_amd.silu_mul_quant(F, torch.randn(2 * F, generator=gen, device="cuda"), xq_d)

    def matmuls_only(st):  # the token's four products with the same fusions
        for t in keep:
            ane_amd.q8_0_matvec_fused(nqkv, H, xin, t["w_qkv"], scratch, norm_w=t["attn_norm"], eps=1e-5, stream=st)
            ane_amd.q8_0_matvec_q8(H, NH * HD, xq_o, t["w_o"], resid, residual=resid, stream=st)
            ane_amd.q8_0_gate_up_silu_quant(F, H, xin, t["ffn_norm"], t["w_gate_up"], xq_g, eps=1e-5, stream=st)
            ane_amd.q8_0_matvec_q8(H, F, xq_d, t["w_down"], resid, residual=resid, stream=st)

    tok_ms = graph_time(token, 3)
    mm_ms = graph_time(matmuls_only, 3)
    kv_bytes = nl * 2 * NKV * CTX * HD * 2
    tok_s = 1e3 / tok_ms
    log(f"decode (config 5, {nl} layers, ctx {CTX}): {tok_ms * 1e3:.1f} us/token = {tok_s:.1f} tok/s; "
        f"mul_mat {mm_ms * 1e3:.1f} us ({mm_ms / tok_ms:.1%}); weights+KV {(wbytes + kv_bytes) / tok_ms / 1e6:.0f} GB/s")
    res = {"workload": f"config 5: decode 1 token, Llama-3-8B shapes, {nl} layers, Q8_0 weights, fp16 KV ctx {CTX}",
           "route": "fused: ane_decode_token (6 launches per layer, the steps fused into the products)",
           "tok_s": round(tok_s, 1), "us_per_token": round(tok_ms * 1e3, 1),
           "mul_mat_us": round(mm_ms * 1e3, 1), "mul_mat_share": round(mm_ms / tok_ms, 4),
           "weights_bytes": int(wbytes), "kv_bytes": int(kv_bytes),
           "GB_s_weights_plus_kv": round((wbytes + kv_bytes) / tok_ms / 1e6, 1),
           "upper_bound_tok_s_at_8TBs": round(8e12 / (wbytes + kv_bytes), 1)}

    # The same model through the ggml hook: each layer's four products are
    # GGML_OP_MUL_MAT nodes run by ane_ggml_compute_forward, the steps around
    # them separate kernels.  mul_mat share = a graph of the token's MUL_MAT
    # nodes alone (same shapes, same backend) / the whole token.
    be = ane_amd.GgmlBackend()
    ws_g = ane_amd.decode_ggml_workspace(cfg)
    T, Gop = ane_amd.GgmlType, ane_amd.GgmlOp
    col_h = torch.randn(H, generator=gen, device="cuda")
    col_f = torch.randn(F, generator=gen, device="cuda")
    col_q = torch.randn(NH * HD, generator=gen, device="cuda")
    out_big = torch.empty(2 * F, device="cuda")
    nodes = []
    for t in keep:
        for W, N_, K_, xcol in ((t["w_qkv"], nqkv, H, col_h), (t["w_o"], H, NH * HD, col_q),
                                (t["w_gate_up"], 2 * F, H, col_h), (t["w_down"], H, F, col_f)):
            wt = ane_amd.ggml_tensor(T.Q8_0, [K_, N_], W)
            xt = ane_amd.ggml_tensor(T.F32, [K_, 1], xcol)
            nodes.append((wt, xt, ane_amd.ggml_tensor(T.F32, [N_, 1], out_big, op=Gop.MUL_MAT, src=(wt, xt))))
    routes = {}
    for name, arith, mode in (("build", ane_amd.ARITH_BUILD, 0), ("reference", ane_amd.ARITH_REFERENCE, 1)):
        def token_g(st, arith=arith):
            be.set_stream(st)
            ane_amd.decode_token_ggml(cfg, layers, table, pos, x, ws_g, be, arith)

        def mul_mats(st, mode=mode):
            be.set_stream(st)
            be.L.ane_ggml_backend_set_q8_mode(be.h, mode)
            for n in nodes:
                be.compute(n[2])

        g_ms = graph_time(token_g, 3)
        gm_ms = graph_time(mul_mats, 3)
        routes[name] = {"tok_s": round(1e3 / g_ms, 1), "us_per_token": round(g_ms * 1e3, 1),
                        "mul_mat_us": round(gm_ms * 1e3, 1), "mul_mat_share": round(gm_ms / g_ms, 4),
                        "q8_0_mode": "G (int8 dots)" if mode == 0 else "R (opcode 0x57 arithmetic)"}
        log(f"decode via the ggml hook, {name} arithmetic: {g_ms * 1e3:.1f} us/token = {1e3 / g_ms:.1f} tok/s; "
            f"MUL_MAT nodes {gm_ms * 1e3:.1f} us ({gm_ms / g_ms:.1%})")
    res["ggml_route"] = {
        "how": "ane_decode_token_ggml: per layer 4 GGML_OP_MUL_MAT nodes (qkv, o, gate|up, down) through "
               "ane_ggml_compute_forward, plus RMSNorm, RoPE + KV append, attention, SiLU*up and residual "
               "kernels; 'build' is bit-identical to the fused route, 'reference' runs the handlers' arithmetic",
        **routes}
    be.close()
    del keep, nodes
    torch.cuda.empty_cache()
    return res


def bench_qformats(args) -> dict:
    """The other weight formats' R-mode GEMVs (q4_0, q4_k, q2_k, q3_k, q5_k,
    q6_k) at 14336x4096, rotating weight copies past the Infinity Cache.
    GB/s counts the weight bytes once plus x and y."""
    import numpy as np
    import torch

    import ane_amd
    from tests import data

    Nr, Kc = 14336, 4096
    x = torch.from_numpy(data.activations(1, Kc, seed=4)[0]).cuda()
    y = torch.empty(Nr, device="cuda", dtype=torch.float32)
    res = {}
    for fmt, (bb, nv) in ane_amd.QFORMATS.items():
        W0 = torch.from_numpy(data.q_weights(fmt, Nr, Kc, seed=3)).cuda()
        wbytes = W0.numel()
        copies = max(2, int(np.ceil(300e6 / wbytes)))
        Ws = [W0] + [W0.clone() for _ in range(copies - 1)]
        it = [0]

        def fn(st):
            W = Ws[it[0] % copies]
            it[0] += 1
            ane_amd.q_gemv(fmt, Nr, Kc, x, W, y, stream=st)

        ms = graph_time(fn, 2 * copies)
        alg = wbytes + 4 * (Kc + Nr)
        gbs = alg / ms / 1e6
        res[fmt] = {"us": round(ms * 1e3, 2), "weights_bytes": wbytes, "GB_s": round(gbs, 1),
                    "frac_hbm": round(gbs / PEAK_HBM_GBS, 4)}
        log(f"{fmt}_gemv {Nr}x{Kc}: {ms * 1e3:.2f} us = {gbs:.0f} GB/s ({gbs / PEAK_HBM_GBS:.1%})")
        del Ws, W0
        torch.cuda.empty_cache()
    return {"workload": f"R-mode GEMV {Nr}x{Kc} per weight format, fp32 x", "shapes": res}


def bench_m_sweep(args, N, K) -> dict:
    """Config 2's M sweep: whole dense_fused_i8 (quantize + contraction) at
    M in {1, 16, 128, 1024}, N = K = 4096."""
    import torch

    import ane_amd

    out = {}
    for M in (1, 16, 128, 1024):
        g = torch.Generator(device="cuda")
        g.manual_seed(2)
        A = torch.randn((M, K), generator=g, device="cuda", dtype=torch.float32)
        B = torch.randn((K, N), generator=g, device="cuda", dtype=torch.float32)
        C = torch.empty((M, N), device="cuda", dtype=torch.float32)
        ws = torch.empty(ane_amd.dense_fused_i8_workspace_size(M, N, K), dtype=torch.uint8, device="cuda")

        def fn(st):
            ane_amd.dense_fused_i8(M, N, K, 1.0, True, A, B, C, workspace=ws, stream=st, check_wait=False)

        ms = graph_time(fn, 20)
        ane_amd.dense_fused_i8_status(ws)
        ops = 2.0 * M * N * K
        alg = 4.0 * (M * K + K * N + M * N)
        out[f"M{M}"] = {"us": round(ms * 1e3, 2), "TOPS": round(ops / ms / 1e9, 2),
                        "GB_s_fp32_io": round(alg / ms / 1e6, 1)}
        log(f"dense_fused_i8 M={M}: {ms * 1e3:.2f} us = {ops / ms / 1e9:.1f} TOPS")
    return {"workload": "config 2 M sweep: dense_fused_i8 M x 4096 x 4096, whole op", "shapes": out}


def bench_igemm(args) -> dict:
    """cblas_igemm (opcode 0x61, the handler's arithmetic) at 1024^3 with
    transB: int8 A (1024 x 1024), int8 B stored N x K, fp32 C, alpha 1,
    beta 0, on the kernel ABI, HIP-graph replayed."""
    import torch

    import ane_amd

    M = N = K = 1024
    g = torch.Generator(device="cuda")
    g.manual_seed(9)
    A = torch.randint(-127, 128, (M, K), generator=g, device="cuda", dtype=torch.int8)
    B = torch.randint(-127, 128, (N, K), generator=g, device="cuda", dtype=torch.int8)
    C = torch.zeros((M, N), device="cuda", dtype=torch.float32)
    ws = torch.empty(max(1, int(ane_amd.lib().ane_hip_cblas_igemm_workspace_size(M, N, K))), dtype=torch.uint8,
                     device="cuda")

    def fn(st):
        ane_amd.cblas_igemm("igemm", 2, M, N, K, K, K, N, 1.0, 0.0, A, B, C, workspace=ws, stream=st)

    ms = graph_time(fn, 50)
    ops = 2.0 * M * N * K
    log(f"cblas_igemm 1024^3 transB: {ms * 1e3:.2f} us = {ops / ms / 1e9:.1f} TOPS")
    return {"workload": "cblas_igemm (0x61) 1024^3, transB, alpha 1, beta 0, handler arithmetic",
            "us": round(ms * 1e3, 3), "TOPS": round(ops / ms / 1e9, 2),
            "frac_int8_peak": round(ops / ms / 1e9 / PEAK_INT8_TOPS, 4)}


def _host_threads() -> int:
    """Host threads for the all-core rows: the CPUs this process may run on,
    capped by OMP_NUM_THREADS (the GPU box sets it to its per-GPU CPU share)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    cap = os.environ.get("OMP_NUM_THREADS")
    if cap and cap.isdigit() and int(cap) > 0:
        n = min(n, int(cap))
    return max(1, n)


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _timed(fn, min_s: float = 1.0, reps: int = 3):
    """Median seconds per call over >= reps calls and >= min_s in total."""
    ts = []
    t_all = time.perf_counter()
    while len(ts) < reps or time.perf_counter() - t_all < min_s:
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
        if len(ts) >= 50:
            break
    ts.sort()
    return ts[len(ts) // 2]


def cpu_baseline(A, B, C, M, N, K) -> dict:
    """The scalar CPU restatement (oracle/, -O2 -ffp-contract=off, OpenMP over
    output rows) on the host cores, for configs 1-4 at 1 thread and at every
    thread this process may use.  Config 2's 4096^3 rows are a bounded sample
    (about 4 s per thread count), extrapolated to the whole op; the sampled
    rows are compared bit for bit with the GPU's C.  `value` is config 2 at
    all threads."""
    import numpy as np

    from tests import _oracle, data

    oracle = _oracle.load()
    nth = _host_threads()
    rows_out = []
    Cg = C.cpu().numpy()
    An = A.cpu().numpy()
    Bn = B.cpu().numpy()
    match = True
    cfg2 = {}
    for threads in (1, nth):
        oracle.set_threads(threads)
        t0 = time.perf_counter()
        qA, sa = oracle.quantize_exact(An.ravel())
        qB, sb = oracle.quantize_exact(Bn.ravel())
        t_quant = time.perf_counter() - t0
        s = np.float32(np.float32(sa * sb) * np.float32(1.0))
        done, t_rows, chunk = 0, 0.0, max(8, 8 * threads)
        while done < M and t_rows < 4.0:
            r1 = min(M, done + chunk)
            t1 = time.perf_counter()
            out = oracle.dense_fused_rows(done, r1, N, K, s, True, qA, qB)
            t_rows += time.perf_counter() - t1
            match = match and np.array_equal(Cg[done:r1].view(np.uint32), out.view(np.uint32))
            done = r1
        t_full = t_quant + t_rows * (M / done)
        tops = 2.0 * M * N * K / t_full / 1e12
        cfg2[threads] = tops
        rows_out.append({"config": f"2: dense_fused_i8 {M}x{N}x{K}", "threads": threads, "value": round(tops, 5),
                         "unit": "TOPS", "sample": f"quantize all of A and B ({t_quant:.2f} s) + {done} of {M} rows "
                         f"({t_rows:.2f} s), extrapolated to the whole op"})
        log(f"cpu config 2, {threads} thread(s): {tops:.4f} TOPS ({done} of {M} rows sampled)")

    # config 1: the MNIST-shaped MLP forward through dense_fused_i8
    x, w1, w2 = data.mnist_inputs(seed=1)
    ops1 = 2.0 * 50 * (784 * 128 + 128 * 10)
    for threads in (1, nth):
        oracle.set_threads(threads)

        def mlp():
            h = oracle.dense_fused_i8(50, 128, 784, np.float32(1.0), True, x, w1)
            oracle.dense_fused_i8(50, 10, 128, np.float32(1.0), False, h, w2)

        sec = _timed(mlp)
        rows_out.append({"config": "1: MNIST MLP 50x784->128 ReLU ->10", "threads": threads,
                         "value": round(sec * 1e6, 1), "unit": "us per forward", "TOPS": round(ops1 / sec / 1e12, 6),
                         "sample": "whole forward, median of >= 3 runs and >= 1 s"})

    # config 3: Q8_0 matvec 14336x4096, R mode (opcode 0x57) and G mode
    Nq, Kq = 14336, 4096
    Wq = data.q8_0_weights(Nq, Kq, seed=3)
    xq = data.activations(1, Kq, seed=4)
    wbytes = Nq * (Kq // 32) * 34 + 4 * (Nq + Kq)
    for threads in (1, nth):
        oracle.set_threads(threads)
        for mode, fn in (("R", lambda: oracle.q8_0_gemv(Nq, Kq, xq[0], Wq)),
                         ("G", lambda: oracle.q8_0_mul_mat_g(Nq, Kq, 1, xq, Wq))):
            sec = _timed(fn)
            rows_out.append({"config": f"3: Q8_0 matvec {Nq}x{Kq} {mode} mode", "threads": threads,
                             "value": round(wbytes / sec / 1e9, 2), "unit": "GB/s",
                             "us": round(sec * 1e6, 1), "sample": "whole matvec, median of >= 3 runs and >= 1 s"})

    # config 4: Q8_0 mul_mat at the four projections, T tokens (bounded: one call each)
    proj = {"qkv": (6144, 4096), "o": (4096, 4096), "gate_up": (28672, 4096), "down": (4096, 14336)}
    for threads in (1, nth):
        oracle.set_threads(threads)
        for T in (1, 4, 16, 64):
            tot_s, tot_ops = 0.0, 0.0
            for name, (Np, Kp) in proj.items():
                if threads == 1 and T > 4:
                    continue  # the 1-thread rows stop at 4 tokens to stay bounded
                W = data.q8_0_weights(Np, Kp, seed=Np + Kp + 1)
                xs = data.activations(T, Kp, seed=T + 200)
                t0 = time.perf_counter()
                oracle.q8_0_mul_mat_g(Np, Kp, T, xs, W)
                tot_s += time.perf_counter() - t0
                tot_ops += 2.0 * Np * Kp * T
            if tot_s:
                rows_out.append({"config": f"4: Q8_0 mul_mat T={T}, qkv+o+gate_up+down", "threads": threads,
                                 "value": round(tot_ops / tot_s / 1e12, 5), "unit": "TOPS",
                                 "us": round(tot_s * 1e6, 1), "sample": "one call per projection"})
    oracle.set_threads(1)
    model = _cpu_model()
    log(f"cpu baseline: {model}, {nth} threads; config 2 {cfg2[nth]:.4f} TOPS ({cfg2[1]:.4f} at 1 thread); "
        f"sampled rows bit-identical to the GPU: {match}")
    return {"value": round(cfg2[nth], 5), "unit": "TOPS", "cores": nth, "kind": "port",
            "cpu_model": model,
            "sample": f"oracle/ane_oracle.c (-O2 -ffp-contract=off, OpenMP over output rows) on config 2 "
                      f"({M}x{N}x{K}): quantize all of A and B + a bounded sample of the contraction's rows "
                      f"(about 4 s), extrapolated to the whole op; every config's rows in 'rows'",
            "gpu_rows_bit_identical": bool(match),
            "rows": rows_out}


if __name__ == "__main__":
    sys.exit(main())
