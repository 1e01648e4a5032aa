#!/usr/bin/env python3
"""Paged-attention decode benchmark on one MI355X (gfx950).

One step = one decode call over the whole batch of the workload, inputs resident in HBM, in the form
the workload's dispatch entry selects (launch.merge): "reduce" -- the partition kernel followed by the
partition-reduce kernel -- or "fused" -- the partition kernel alone, its last workgroup per sequence
and head slot merging the partition records.  --merge overrides the entry.  The library runs the
partition kernel on the work-queue schedule when the call's work items exceed the workgroups the GPU
holds at once (config.schedule; the kernel is then pa_partition_queue_kernel, whose ticket counter
resets itself in the fused form and is zeroed by a one-thread kernel in front of it in the reduce
form), else one workgroup per work item.  Default workload: 128 sequences, 32 query / 8 KV heads,
head_dim 128, block 16, bf16, context lengths ~ U[1024, 16384] (seeded), 4.24 GB of K/V per call --
about 16x the 256 MB last-level cache, so every call streams from HBM.

Timing: every form below is timed as S (--samples, default 10) interleaved samples of K (--steps)
back-to-back launches, each sample bracketed by synchronisations and HIP events on the launch
stream; consecutive samples run the forms in opposite orders.  Reported figures are medians over
the samples; timing.cv_pct_events is the headline form's coefficient of variation.

Prints one JSON line:
  value            effective KV GB/s = algorithmic K+V bytes per call / wall time per call
  us_per_call      median wall time per call of the headline form: K whole calls back to back,
                   nothing else on the stream (us_per_call_events: the same samples by HIP events)
  roofline         the partition kernel against the 8 TB/s HBM peak: achieved = KV bytes / its
                   median duration by HIP events (in the fused form the call is that one kernel);
                   traffic = measured
                   HBM bytes per launch from the committed rocprofv3 counter summary for this exact
                   configuration (null when there is none)
  kernels_us       per-launch averages of the reduce form's two kernels; us_per_call_reduce and
                   us_per_call_fused time both whole-call forms (omitted with --no-breakdown, which
                   times the headline form only)
  cpu_baseline     the reference algorithm (its torch fallback, restated in oracle/) on the host
                   cores over a bounded sample of the same workload

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--samples S] [--workload c5] [--variant mfma]
                       [--partition P] [--merge fused|reduce] [--schedule auto|grid|queue]
                       [--no-breakdown] [--no-cpu-baseline]
                       [--cpu-seconds S] [--calibration-copy]
       python bench.py --operator kv_cache_append|kv_cache_copy [--case ...] [--dtype bf16]
                       (the paged-cache operators around the decode; same JSON line shape)
       python bench.py --operator sdpa [--case ...] [--dtype bf16]
                       (prefill self-attention; roofline against the dense MFMA peak)
"""

from __future__ import annotations

import argparse
import json
import math
import os
import re
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for entry in (str(ROOT / "radeon-kernels_amd"), str(ROOT)):
    if entry not in sys.path:
        sys.path.insert(0, entry)

HBM_PEAK_GBPS = 8000.0
METRIC = "paged-attn decode µs/call + effective KV GB/s (% MI355X HBM peak), b128"
# Committed counter summaries of the partition kernel: the 128-sequence workload on either schedule and
# the small workloads; each names the exact configuration it measured.
TRAFFIC_SUMMARIES = (ROOT / "profiles" / "pa_partition_queue_kernel_b128_traffic.txt",
                     ROOT / "profiles" / "pa_partition_kernel_b128_traffic.txt",
                     *sorted((ROOT / "profiles").glob("pa_partition_kernel_*_counters.txt")))


def parse_args(argv=None):
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--samples", type=int, default=10,
                        help="interleaved samples of --steps calls per timed form (medians reported)")
    parser.add_argument("--workload", default="c5",
                        help="c1..c5 (the five measured shapes) or one of the reference's decode cases, "
                             "<case id>-<fp16|bf16> (benchmarks/workloads/paged_attention_decode-1.0.yaml)")
    parser.add_argument("--variant", default=None, choices=["mfma", "valu", "mfma_qk"])
    parser.add_argument("--partition", type=int, default=None)
    parser.add_argument("--merge", default=None, choices=["fused", "reduce"],
                        help="partition-record merge form (default: the workload's dispatch entry)")
    parser.add_argument("--schedule", default="auto", choices=["auto", "grid", "queue"],
                        help="partition-kernel schedule (default: the library's choice)")
    parser.add_argument("--no-breakdown", action="store_true",
                        help="time only the headline call (no per-kernel breakdown of the other form)")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-rk-call", action="store_true",
                        help="skip timing the public operator (rk_call), e.g. under a profiler")
    parser.add_argument("--append", action="store_true",
                        help="paged_attention_decode: also time one serving step that first appends each "
                             "sequence's new token (position context_length - 1): kv_cache_append then the "
                             "decode (two launches) against rk_pa_decode_append (one launch)")
    parser.add_argument("--cpu-seconds", type=float, default=12.0)
    parser.add_argument("--calibration-copy", action="store_true",
                        help="run a 1 GiB device copy before timing (counter calibration under rocprofv3)")
    parser.add_argument("--operator", default="paged_attention_decode",
                        choices=["paged_attention_decode", "kv_cache_append", "kv_cache_copy", "sdpa"])
    parser.add_argument("--case", default=None,
                        help="kv_cache_append / kv_cache_copy / sdpa case (benchmarks/workloads/<operator>-1.0.yaml "
                             "in the reference, or an sdpa long-prefill case); defaults: prefill-t128-mha32-d128-p32, "
                             "beam-pairs64-gqa8-d256-p16, b4-gqa32x8-s4096-d128-causal")
    parser.add_argument("--dtype", default="bf16", choices=["fp16", "bf16"],
                        help="element type of the KV-cache and sdpa operators")
    return parser.parse_args(argv)


PUBLIC_CALLS_MIN = 200


def public_call_us(torch, call, steps: int, batches: int = 5) -> float:
    """Host wall time per call of the public operator: the median of ``batches`` batches of ``steps``
    (at least PUBLIC_CALLS_MIN) back-to-back calls, each batch closed by a synchronisation (single
    batches were seen to catch one-off host stalls of the machine; batches of 10 calls added the two
    synchronisations, 2-3 us, to every microsecond-scale call)."""

    import statistics

    steps = max(steps, PUBLIC_CALLS_MIN)
    times = []
    for _ in range(batches):
        torch.cuda.synchronize()
        t = time.perf_counter()
        for _ in range(steps):
            call()
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t) / steps * 1e6)
    return statistics.median(times)


SETTLE_SECONDS = 0.1


def settle(torch, launch, copies: int = 1, seconds: float = SETTLE_SECONDS, limit: int = 100000) -> None:
    """Untimed launches for at least ``seconds`` (at most ``limit`` rounds) before the warmup steps.

    A few warmup steps of a microsecond-scale call leave the GPU's clocks still ramping when the timed
    region starts; the first timed region of the b1 decode then measured about 0.9 us per call slower
    than an identical later one.  ``launch(i)`` runs on input copy ``i % copies``, rotating as the timed
    loops do, so a kernel trace of the run averages one kind of launch.
    """

    torch.cuda.synchronize()
    start = time.perf_counter()
    i = 0
    for _ in range(limit):
        for _ in range(10):
            launch(i % copies)
            i += 1
        torch.cuda.synchronize()
        if time.perf_counter() - start >= seconds:
            break


def dispatch_launch(torch, q, k, v, bt, cl) -> dict:
    """The dispatch decision of the public operator on these inputs (entry id, entrypoint, launch
    parameters), from one call that must run natively."""

    import warnings

    import radeon_kernels as rk
    from radeon_kernels.ops._runtime import NativeDemotionWarning

    with warnings.catch_warnings():
        # A demotion would run the torch fallback (tens of GB of intermediates on the largest workload).
        warnings.simplefilter("error", NativeDemotionWarning)
        rk.paged_attention_decode(q, k, v, bt, cl)
    torch.cuda.synchronize()
    return rk.get_last_dispatch()


def read_traffic(workload: str, variant: str, partition: int, merge: str, schedule: str, kv_bytes: int,
                 seed: int | None = None):
    """HBM bytes per partition-kernel launch from a committed counter summary, if one was measured
    on exactly this configuration: workload, variant, partition size, merge form, schedule and the
    same input draw (its KV bytes per call, and its seed where the summary records one)."""

    found = read_summary(workload, variant, partition, merge, schedule, kv_bytes, seed)
    return None if found is None else found[1]


def read_summary(workload: str, variant: str, partition: int, merge: str, schedule: str, kv_bytes: int,
                 seed: int | None = None):
    """(summary path, HBM bytes per launch, kernel-trace average in us or None) of the committed counter
    summary measured on exactly this configuration, or None."""

    for summary in TRAFFIC_SUMMARIES:
        if not summary.is_file():
            continue
        fields = {}
        for line in summary.read_text().splitlines():
            if "=" in line and not line.lstrip().startswith("#"):
                key, value = line.split("=", 1)
                fields[key.strip()] = value.strip()
        try:
            if (fields.get("workload") == workload and fields.get("variant") == variant
                    and int(fields["partition_tokens"]) == partition and fields.get("merge", "reduce") == merge
                    and fields.get("schedule", "grid") == schedule and int(fields["kv_bytes_per_call"]) == kv_bytes
                    and ("seed" not in fields or seed is None or int(fields["seed"]) == seed)):
                average = re.search(r"dispatches, average ([0-9.]+) us", summary.read_text())
                return summary, int(fields["hbm_bytes_per_launch"]), float(average.group(1)) if average else None
        except (KeyError, ValueError):
            continue
    return None


PHASE_SYMBOL = {"all": "rk_pa_decode", "fused": "rk_pa_decode_fused"}


def calibration_copy(torch, device) -> None:
    """One 1 GiB device-to-device copy: under rocprofv3 --pmc its FETCH_SIZE / WRITE_SIZE readings
    against the 1 GiB it is known to read and write give the counters' scale factors."""

    src = torch.empty(1 << 30, dtype=torch.uint8, device=device).fill_(1)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def read_case_traffic(summary: Path, workload: str):
    """HBM bytes per kernel launch from a committed counter summary of one kv-cache or sdpa case, if
    the summary's ``workload`` (operator, case and dtype) is exactly this run's."""

    if not summary.is_file():
        return None
    fields = {}
    for line in summary.read_text().splitlines():
        if "=" in line and not line.lstrip().startswith("#"):
            key, value = line.split("=", 1)
            fields[key.strip()] = value.strip()
    try:
        return int(fields["hbm_bytes_per_launch"]) if fields.get("workload") == workload else None
    except (KeyError, ValueError):
        return None


def cpu_threads() -> tuple[int, int]:
    """(threads used, cores in this process's affinity mask).  The thread count is the affinity mask,
    capped by OMP_NUM_THREADS where the machine sets it to the job's CPU share."""

    affinity = len(os.sched_getaffinity(0))
    share = os.environ.get("OMP_NUM_THREADS", "")
    threads = min(affinity, int(share)) if share.isdigit() and int(share) > 0 else affinity
    return threads, affinity


def cpu_baseline(torch, data, seconds: float) -> dict:
    """The reference algorithm (its torch fallback, restated in oracle/) on the host cores.

    Protocol: torch's CPU thread count is set to ``cpu_threads()``; the sample is the first
    sequences of the workload whose rows one pass covers in about ``seconds / 4`` (the whole batch
    for the small workloads), evaluated two sequences at a time; one untimed warmup pass, then three
    timed passes (more for passes under 0.5 s, up to ``seconds`` in total and 30 passes); the reported rate is the
    median pass.  K/V rows of the sample are gathered on the device and copied to the host before
    timing, so the timed region is the fallback alone.
    """

    import statistics

    from oracle import pa_oracle

    threads, affinity = cpu_threads()
    torch.set_num_threads(threads)
    w = data["workload"]
    bt_all = data["block_tables"].cpu().to(torch.int64)
    ctx_all = data["context_lengths"].cpu().to(torch.int64)
    batch = bt_all.shape[0]
    cap = w.max_blocks * w.block_size
    chunk = 2

    def prepared_chunk(rows):
        bt, ctx = bt_all[rows], ctx_all[rows]
        need = [min(math.ceil(int(c) / w.block_size), w.max_blocks) for c in ctx]
        used = torch.cat([bt[i, : need[i]] for i in range(len(rows))])
        remap = {int(b): i for i, b in enumerate(used.tolist())}
        compact = torch.zeros_like(bt)
        for i in range(len(rows)):
            compact[i, : need[i]] = torch.tensor([remap[int(b)] for b in bt[i, : need[i]]])
        index = used.to(data["key_cache"].device)
        return (data["query"][rows].cpu(), data["key_cache"].index_select(0, index).cpu(),
                data["value_cache"].index_select(0, index).cpu(), compact.to(torch.int32), ctx.to(torch.int32))

    def run(chunks) -> float:
        start = time.perf_counter()
        for q, k, v, bt, ctx in chunks:
            pa_oracle.fallback_restated(torch, q, k, v, bt, ctx)
        return time.perf_counter() - start

    # Size the sample: add chunks until one untimed pass over them takes seconds / 4 (this pass is
    # the warmup).
    chunks, warm, done = [], 0.0, 0
    while done < batch and warm < seconds / 4:
        rows = list(range(done, min(batch, done + chunk)))
        prepared = prepared_chunk(rows)
        warm += run([prepared])
        chunks.append(prepared)
        done += len(rows)
    tokens = int(sum(min(int(c), cap) for c in ctx_all[:done]))
    kv = tokens * w.kv_heads * w.head_dim * 2 * w.elem_size
    passes = [run(chunks) for _ in range(3)]
    while sum(passes) + warm < seconds and statistics.median(passes) < 0.5 and len(passes) < 30:
        passes.append(run(chunks))
    per_pass = statistics.median(passes)
    gbps = kv / per_pass / 1e9
    info = torch.__config__.parallel_info().splitlines()
    return {
        "value": round(gbps, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"first {done} of {batch} sequences ({tokens} context tokens, {kv / 1e9:.4f} GB of K/V) per "
                   f"pass, {chunk} sequences at a time, by the reference's torch fallback restated in "
                   f"oracle/pa_oracle.py (torch {torch.__version__} CPU, {threads} threads); 1 warmup pass, "
                   f"median of {len(passes)} timed passes"),
        "pass_seconds": {"passes": len(passes), "median": round(per_pass, 4), "min": round(min(passes), 4),
                         "max": round(max(passes), 4)},
        "affinity_cores": affinity,
        "parallel_info": [line.strip() for line in info if line.strip()][:8],
        "us_per_call_extrapolated": round(data["kv_bytes"] / (gbps * 1e9) * 1e6, 1),
    }


MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 / fp16 MFMA


def main_sdpa(args) -> int:
    """``--operator sdpa``: one step = one self-attention forward call of the case (one kernel)."""

    import torch

    from radeon_kernels.cabi import sdpa_library
    from benchmarks.workloads import SDPA_CASES, SDPA_LONG_CASES, make_sdpa_inputs

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no visible ROCm GPU"}))
        return 1
    device = torch.device("cuda:0")
    lib = sdpa_library()  # raises if the HIP library was not built
    if args.calibration_copy:
        calibration_copy(torch, device)
    cases = {**SDPA_CASES, **SDPA_LONG_CASES}
    case = cases[args.case or "b4-gqa32x8-s4096-d128-causal"]
    data = make_sdpa_inputs(case, dtype=args.dtype, device=device, generator_device=device)
    q, k, v = data["query"], data["key"], data["value"]
    scale = 1.0 / math.sqrt(case.head_dim)
    out = torch.empty_like(q)
    stream = torch.cuda.current_stream(device)

    # Arguments converted once: one foreign call per launch, so small cases time the GPU.
    launch = lib.prepare_forward(q, k, v, is_causal=case.causal, scale=scale, out=out, stream=stream)

    settle(torch, lambda _: launch())
    for _ in range(args.warmup):
        launch()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t = time.perf_counter()
    start.record(stream)
    for _ in range(args.steps):
        launch()
    end.record(stream)
    torch.cuda.synchronize()
    us_per_call = (time.perf_counter() - t) / args.steps * 1e6
    kernel_us = start.elapsed_time(end) * 1e3 / args.steps
    flops = case.flops()

    import warnings

    import radeon_kernels as rk
    from radeon_kernels.ops._runtime import NativeDemotionWarning

    with warnings.catch_warnings():
        warnings.simplefilter("error", NativeDemotionWarning)
        rk.sdpa(q, k, v, is_causal=case.causal)
    decision = rk.get_last_dispatch()
    rk_us = public_call_us(torch, lambda: rk.sdpa(q, k, v, is_causal=case.causal), max(1, args.steps // 5))
    # The operator's declared fallback on the same GPU (torch's scaled_dot_product_attention).
    from radeon_kernels.ops.sdpa.reference import sdpa_fallback

    fallback_us = public_call_us(torch, lambda: sdpa_fallback(torch, q, k, v, case.causal, scale),
                                 max(1, args.steps // 5))
    result = {
        "metric": "sdpa prefill TFLOP/s over attended (query, key) pairs (% MI355X dense MFMA peak)",
        "value": round(flops / (us_per_call * 1e6), 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_per_call / 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic (seeded N(0,1) query/key/value)",
        "config": {
            "workload": f"sdpa-{case.key}-{args.dtype}", "batch": case.batch, "query_heads": case.query_heads,
            "kv_heads": case.kv_heads, "sequence": case.sequence, "head_dim": case.head_dim,
            "causal": case.causal, "reference_case": case.key in SDPA_CASES,
            "arch": torch.cuda.get_device_properties(0).gcnArchName.split(":", 1)[0],
        },
        "us_per_call": round(us_per_call, 2),
        "flops_per_call": flops,
        "kernels_us": {"sdpa_fwd_kernel": round(kernel_us, 2)},
        "roofline": {
            "bound": "mfma",
            "achieved": round(flops / (kernel_us * 1e6), 2),
            "peak": MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(flops / (kernel_us * 1e6) / MFMA_PEAK_TFLOPS, 4),
            "traffic": read_case_traffic(ROOT / "profiles" / f"sdpa_fwd_kernel_{case.key}_traffic.txt",
                                         f"sdpa-{case.key}-{args.dtype}"),
        },
        "rk_call": {"us_per_call": round(rk_us, 2), "selected": decision["selected"], "entry_id": decision["entry_id"]},
        "torch_sdpa_fallback_us": round(fallback_us, 2),
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline_sdpa(torch, case, data, min(args.cpu_seconds,
                                                                                                    10.0)),
    }
    print(json.dumps(result), flush=True)
    return 0


def cpu_baseline_sdpa(torch, case, data, seconds: float) -> dict:
    """The reference's explicit fp32 evaluation (restated in oracle/) on the host cores, one
    (sequence, query head) slice at a time, for about ``seconds``; reported per whole call."""

    from oracle import sdpa_oracle

    q, k, v = (data[n].cpu() for n in ("query", "key", "value"))
    group = case.query_heads // case.kv_heads
    scale = 1.0 / math.sqrt(case.head_dim)
    slices = [(b, h) for b in range(case.batch) for h in range(case.query_heads)]
    done, t = 0, time.perf_counter()
    while done < len(slices) and time.perf_counter() - t < seconds:
        b, h = slices[done]
        sdpa_oracle.fallback_restated(torch, q[b:b + 1, h:h + 1], k[b:b + 1, h // group:h // group + 1],
                                      v[b:b + 1, h // group:h // group + 1], case.causal, scale)
        done += 1
    elapsed = time.perf_counter() - t
    per_call = elapsed / done * len(slices)
    return {"value": round(case.flops() / (per_call * 1e12), 4), "unit": "TFLOP/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{done} of {len(slices)} (sequence, query head) slices of the explicit fp32 reference "
                      f"(oracle/sdpa_oracle.py, torch {torch.__version__} CPU), {elapsed:.1f} s",
            "us_per_call_extrapolated": round(per_call * 1e6, 1)}


def main_kv(args) -> int:
    """``--operator kv_cache_append|kv_cache_copy``: one step = one call of the case (one kernel)."""

    import torch

    from radeon_kernels.cabi import kv_library
    from benchmarks.workloads import APPEND_CASES, COPY_CASES, make_append_inputs, make_copy_inputs

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no visible ROCm GPU"}))
        return 1
    device = torch.device("cuda:0")
    lib = kv_library()  # raises if the HIP library was not built
    if args.calibration_copy:
        calibration_copy(torch, device)
    if args.operator == "kv_cache_append":
        case = APPEND_CASES[args.case or "prefill-t128-mha32-d128-p32"]
        data = make_append_inputs(case, dtype=args.dtype, index_dtype="int64", device=device)
        names = ("key", "value", "key_cache", "value_cache", "slot_mapping")
        moved = case.bytes_moved() + case.tokens * 8  # K/V rows read and written, plus the slots
        prepare, kernel = lib.prepare_append, "kv_append_kernel"
        shape = {"tokens": case.tokens}
    else:
        case = COPY_CASES[args.case or "beam-pairs64-gqa8-d256-p16"]
        data = make_copy_inputs(case, dtype=args.dtype, index_dtype="int64", device=device)
        names = ("key_cache", "value_cache", "block_mapping")
        moved = case.bytes_moved() + case.pairs * 16  # K/V blocks read and written, plus the mapping
        prepare, kernel = lib.prepare_copy, "kv_copy_kernel"
        shape = {"pairs": case.pairs}
    cache_bytes = data["key_cache"].numel() * 2 * 2
    # The caches fit in the 256 MB last-level cache: rotate among enough independent copies of every
    # input that each call's rows come from and go to HBM.
    copies = max(16, math.ceil(768e6 / cache_bytes))
    sets = [tuple(data[n] for n in names)] + [tuple(data[n].clone() for n in names) for _ in range(copies - 1)]
    stream = torch.cuda.current_stream(device)
    # Arguments converted once per input set: one foreign call per launch, so the loop times the GPU.
    launches = [prepare(*inputs, stream=stream) for inputs in sets]
    settle(torch, lambda i: launches[i](), copies)
    for i in range(args.warmup):
        launches[i % copies]()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t = time.perf_counter()
    start.record(stream)
    for i in range(args.steps):
        launches[i % copies]()
    end.record(stream)
    torch.cuda.synchronize()
    us_per_call = (time.perf_counter() - t) / args.steps * 1e6
    kernel_us = start.elapsed_time(end) * 1e3 / args.steps
    torch.cuda.synchronize()
    t = time.perf_counter()
    for _ in range(args.steps):
        launches[0]()
    torch.cuda.synchronize()
    hot = (time.perf_counter() - t) / args.steps * 1e6

    import warnings

    import radeon_kernels as rk
    from radeon_kernels.ops._runtime import NativeDemotionWarning

    public = rk.kv_cache_append if args.operator == "kv_cache_append" else rk.kv_cache_copy
    with warnings.catch_warnings():
        warnings.simplefilter("error", NativeDemotionWarning)
        public(*sets[0])
    decision = rk.get_last_dispatch()
    rk_us = public_call_us(torch, lambda: public(*sets[0]), max(1, args.steps // 5))

    result = {
        "metric": f"{args.operator} µs/call + effective GB/s (% MI355X HBM peak)",
        "value": round(moved / (us_per_call * 1e3), 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_per_call / 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic (seeded uniform[-0.5, 0.5) values, unique random slots / disjoint block pairs)",
        "config": {
            "workload": f"{args.operator}-{case.key}-{args.dtype}", **shape, "num_blocks": case.num_blocks,
            "block_size": case.block_size, "kv_heads": case.kv_heads, "head_dim": case.head_dim,
            "index_dtype": "int64", "copies_rotated": copies,
            "arch": torch.cuda.get_device_properties(0).gcnArchName.split(":", 1)[0],
        },
        "us_per_call": round(us_per_call, 2),
        "us_per_call_cache_resident": round(hot, 2),
        "bytes_per_call": moved,
        "kernels_us": {kernel: round(kernel_us, 2)},
        "roofline": {
            "bound": "hbm",
            "achieved": round(moved / (kernel_us * 1e3), 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(moved / (kernel_us * 1e3) / HBM_PEAK_GBPS, 4),
            "traffic": read_case_traffic(ROOT / "profiles" / f"{kernel}_{case.key}.txt",
                                         f"{args.operator}-{case.key}-{args.dtype}"),
        },
        "rk_call": {"us_per_call": round(rk_us, 2), "selected": decision["selected"], "entry_id": decision["entry_id"]},
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline_kv(torch, args.operator, data, moved,
                                                                           min(args.cpu_seconds, 5.0)),
    }
    print(json.dumps(result), flush=True)
    return 0


def cpu_baseline_kv(torch, operator: str, data, moved: int, seconds: float) -> dict:
    """The reference fallback's steps (index_select / index_copy_) on CPU copies of the inputs."""

    from oracle import kv_oracle

    threads = torch.get_num_threads()
    if operator == "kv_cache_append":
        cpu = [data[n].cpu() for n in ("key", "value", "key_cache", "value_cache", "slot_mapping")]
        step = lambda: kv_oracle.append_inplace_torch(torch, *cpu)  # noqa: E731
    else:
        cpu = [data[n].cpu() for n in ("key_cache", "value_cache", "block_mapping")]
        step = lambda: kv_oracle.copy_inplace_torch(torch, *cpu)  # noqa: E731
    calls, elapsed = 0, 0.0
    while elapsed < seconds:
        t = time.perf_counter()
        for _ in range(20):
            step()
        elapsed += time.perf_counter() - t
        calls += 20
    us = elapsed / calls * 1e6
    return {
        "value": round(moved / (us * 1e3), 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{calls} calls of the same case on CPU tensors by the reference fallback's torch steps "
                   f"(oracle/kv_oracle.py; torch {torch.__version__}, {threads} threads), {elapsed:.1f} s"),
        "us_per_call": round(us, 2),
    }


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus == 1 and args.operator == "sdpa":
        return main_sdpa(args)
    if args.gpus == 1 and args.operator != "paged_attention_decode":
        return main_kv(args)
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU only; the decode shards by sequence and KV head "
                          "with no exchange, so multi-GPU throughput is N x the single-GPU value and is not measured here",
                          "n_gpus": args.gpus}))
        return 2

    import torch

    from radeon_kernels.cabi import library
    from benchmarks.workloads import WORKLOADS, make_inputs

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no visible ROCm GPU"}))
        return 1
    device = torch.device("cuda:0")
    arch = torch.cuda.get_device_properties(0).gcnArchName.split(":", 1)[0]
    lib = library()  # raises if the HIP library was not built
    if args.workload not in WORKLOADS:
        print(json.dumps({"error": f"unknown workload {args.workload!r}", "workloads": sorted(WORKLOADS)}))
        return 2
    w = WORKLOADS[args.workload]

    if args.calibration_copy:
        calibration_copy(torch, device)

    data = make_inputs(w, device=device)
    decision = dispatch_launch(torch, data["query"], data["key_cache"], data["value_cache"], data["block_tables"],
                               data["context_lengths"])
    variant = args.variant or decision["selected"].split("/", 1)[1].split("_", 1)[1]  # native/decode_<variant>
    partition = args.partition or int(decision["launch"]["partition_tokens"])
    merge = args.merge or str(decision["launch"]["merge"])
    if merge == "auto":  # the broad region's choice: fused
        merge = "fused"
    kv_bytes = data["kv_bytes"]
    cache_bytes = data["key_cache"].numel() * 2 * 2
    # Small workloads fit in the 256 MB last-level cache: rotate among enough K/V copies that each
    # call reads its cache from HBM.
    copies = 1 if w.ragged else max(16, math.ceil(768e6 / cache_bytes))
    caches = [(data["key_cache"], data["value_cache"])]
    for _ in range(copies - 1):
        caches.append((data["key_cache"].clone(), data["value_cache"].clone()))
    q, bt, cl = data["query"], data["block_tables"], data["context_lengths"]
    batch, hq, d = q.shape
    nb, bs, hkv, _ = data["key_cache"].shape
    mb = bt.shape[1]
    need = lib.workspace_bytes(batch, hq, d, bs, mb, partition)
    out = torch.empty_like(q)
    workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=device)
    counters = torch.zeros(lib.counter_words(batch, hq, hkv), dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream(device)
    headline = "fused" if merge == "fused" else "all"
    schedule = lib.schedule(batch, hq, hkv, d, bs, mb, w.dtype, partition, variant, schedule=args.schedule)
    partition_kernel = "pa_partition_queue_kernel" if schedule == "queue" else "pa_partition_kernel"

    # Every launch's ctypes arguments are built once, so a timed loop makes one foreign call per
    # launch: on the small workloads the wrapper's Python would otherwise outrun the GPU time.
    prepared = {}

    def prepare(phase: str) -> None:
        for copy, (k, v) in enumerate(caches):
            if (phase, copy) not in prepared:
                prepared[phase, copy] = lib.prepare(q, k, v, bt, cl, partition_tokens=partition, variant=variant,
                                                    out=out, workspace=workspace, stream=stream, phase=phase,
                                                    counters=counters, schedule=args.schedule)

    def launch(phase: str, copy: int) -> None:
        prepared[phase, copy]()

    prepare(headline)
    settle(torch, lambda i: launch(headline, i), copies)
    for i in range(args.warmup):
        launch(headline, i % copies)
    torch.cuda.synchronize()

    def region(phase: str) -> tuple[float, float]:
        """K back-to-back launches of `phase` bracketed by HIP events on the launch stream.

        Returns (average µs per launch by the events, wall µs per launch by the host clock)."""

        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t = time.perf_counter()
        start.record(stream)
        for i in range(args.steps):
            launch(phase, i % copies)
        end.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t
        return start.elapsed_time(end) * 1e3 / args.steps, wall * 1e6 / args.steps

    # The timed regions.  Every form bench reports is timed as S interleaved samples of K launches,
    # after the reference's protocol of paired, order-alternating samples (benchmark.py:221-229; its
    # workload file asks for 30 samples and a CV of at most 3%,
    # benchmarks/workloads/paged_attention_decode-1.0.yaml:8-11; S defaults to 10 here so the default run
    # stays short, and the headline's CV is reported): sample s runs the headline form (K whole decode
    # calls, nothing else on the stream), then the
    # reduce form's partition kernel and merge kernel alone, then the other whole-call form, and
    # sample s + 1 runs them in the reverse order, so no form always runs first.  value, ms_per_step
    # and roofline.frac are medians over the headline samples.  In the fused form the call is the
    # partition kernel alone (its average duration is the roofline figure); the reduce form's
    # roofline figure is its partition kernel.
    phases = [headline]
    if not args.no_breakdown or merge == "reduce":
        phases.append("partitions")
        if need > 0:  # one partition covering every sequence needs no reduce launch
            phases.append("reduce")
    other = "reduce" if merge == "fused" else "fused"
    if not args.no_breakdown:
        phases.append("fused" if other == "fused" else "all")
    for phase in phases:
        prepare(phase)  # outside the timed regions
    samples = {phase: [] for phase in phases}
    for s_index in range(args.samples):
        for phase in (phases if s_index % 2 == 0 else phases[::-1]):
            samples[phase].append(region(phase))

    def median_of(phase: str, which: int) -> float:
        return statistics.median(x[which] for x in samples[phase])

    event_us, us_per_call = median_of(headline, 0), median_of(headline, 1)
    head_events = [x[0] for x in samples[headline]]
    cv_pct = statistics.pstdev(head_events) / statistics.mean(head_events) * 100
    part_avg = median_of("partitions", 0) if "partitions" in samples else None
    red_avg = median_of("reduce", 0) if "reduce" in samples else None
    forms = {merge: us_per_call}
    if not args.no_breakdown:
        forms[other] = median_of("fused" if other == "fused" else "all", 1)
    kernel_avg = part_avg if merge == "reduce" else event_us
    gbps = kv_bytes / (us_per_call * 1e3)
    achieved = kv_bytes / (kernel_avg * 1e3)

    hot = None
    if copies > 1:  # the same cache every call: last-level-cache resident
        # HIP events on the launch stream, like the headline figure: a host clock around K = 50
        # microsecond-scale calls also counts the closing synchronisation, about 0.6 us per call.
        hot_samples = []
        for _ in range(3):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            for _ in range(args.steps):
                launch(headline, 0)
            end.record(stream)
            end.synchronize()
            hot_samples.append(start.elapsed_time(end) * 1e3 / args.steps)
        hot = round(statistics.median(hot_samples), 2)

    # The public operator end to end (validation, dispatch, pack lookup, output and workspace
    # allocation, both launches) on the same inputs, back to back.
    import radeon_kernels as rk

    k, v = caches[0]
    rk_us = None if args.no_rk_call else public_call_us(torch, lambda: rk.paged_attention_decode(q, k, v, bt, cl),
                                                           max(1, args.steps // 5))

    step = None
    if args.append:
        # One decode step with its append, both forms, over the same rotating caches (the appends
        # rewrite one slot per sequence of each copy; the decode timings above are already taken).
        from radeon_kernels.cabi import kv_library

        if variant not in ("mfma", "mfma_qk"):
            raise SystemExit("--append needs an mfma variant")
        kvlib = kv_library()
        gen = torch.Generator(device=device).manual_seed(data["seed"] + 1)
        new_k = torch.randn((batch, hkv, d), generator=gen, device=device).to(q.dtype)
        new_v = torch.randn((batch, hkv, d), generator=gen, device=device).to(q.dtype)
        pos = cl.long() - 1  # no slot (-1) for an empty context or one past the table, as the decode treats them
        safe = pos.clamp(min=0, max=mb * bs - 1)
        slots = torch.where((pos >= 0) & (pos < mb * bs),
                            bt.long().gather(1, (safe // bs).unsqueeze(1)).squeeze(1) * bs + safe % bs,
                            torch.full_like(pos, -1))
        appends = [kvlib.prepare_append(new_k, new_v, kc, vc, slots, stream=stream) for kc, vc in caches]
        fused_steps = [lib.prepare(q, kc, vc, bt, cl, partition_tokens=partition, variant=variant, out=out,
                                   workspace=workspace, stream=stream, phase=headline, counters=counters,
                                   new_key=new_k, new_value=new_v, schedule=args.schedule) for kc, vc in caches]

        def step_us(one_step) -> float:
            for i in range(args.warmup):
                one_step(i % copies)
            torch.cuda.synchronize()
            t = time.perf_counter()
            for i in range(args.steps):
                one_step(i % copies)
            torch.cuda.synchronize()
            return (time.perf_counter() - t) / args.steps * 1e6

        def two_launches(i: int) -> None:
            appends[i]()
            launch(headline, i)

        two = step_us(two_launches)
        one = step_us(lambda i: fused_steps[i]())
        step = {"append_tokens": int(batch), "us_per_step_two_launch": round(two, 2),
                "us_per_step_one_launch": round(one, 2), "entrypoints": ["rk_kv_cache_append + " + PHASE_SYMBOL[headline],
                                                                         "rk_pa_decode_append"]}

    summary = read_summary(w.name, variant, partition, merge, schedule, kv_bytes, data["seed"])
    traffic = None if summary is None else summary[1]
    result = {
        "metric": METRIC,
        "value": round(gbps, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_per_call / 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w.dtype,
        "data": ("synthetic (seeded U(-0.125, 0.125) query/K/V as the reference benchmark draws them, seeded block "
                 "tables)" if w.distribution == "uniform" else
                 "synthetic (seeded N(0,1) query/K/V, seeded block tables and context lengths, drawn on the CPU)"),
        "config": {
            "workload": w.name,
            "batch": int(batch), "query_heads": int(hq), "kv_heads": int(hkv), "head_dim": int(d),
            "block_size": int(bs), "num_blocks": int(nb), "max_blocks_per_sequence": int(mb),
            "context": list(w.context) if w.ragged else w.context, "seed": data["seed"],
            "entrypoint": f"decode_{variant}", "partition_tokens": partition, "kv_copies_rotated": copies,
            "merge": merge,
            "schedule": schedule,
            "arch": arch,
        },
        "us_per_call": round(us_per_call, 2),
        "us_per_call_events": round(event_us, 2),
        "timing": {"samples": args.samples, "calls_per_sample": args.steps, "statistic": "median",
                   "interleaved_forms": phases, "cv_pct_events": round(cv_pct, 3),
                   "us_per_call_events_samples": [round(x, 2) for x in head_events]},
        "pct_hbm_peak": round(gbps / HBM_PEAK_GBPS * 100, 2),
        "kv_bytes_per_call": kv_bytes,
        "kernels_us": None if part_avg is None else {
            partition_kernel: round(part_avg, 2),
            "pa_reduce_kernel": None if red_avg is None else round(red_avg, 2)},
        "us_per_call_reduce": round(forms["reduce"], 2) if "reduce" in forms else None,
        "us_per_call_fused": round(forms["fused"], 2) if "fused" in forms else None,
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            # The committed rocprofv3 summary of this configuration (another run, usually another machine):
            # its kernel-trace average and the fraction of peak that average gives.
            "profile": None if summary is None or summary[2] is None else {
                "summary": str(summary[0].relative_to(ROOT)), "kernel_avg_us": summary[2],
                "frac": round(kv_bytes / (summary[2] * 1e3) / HBM_PEAK_GBPS, 4)},
        },
    }
    if hot is not None:
        result["us_per_call_cache_resident"] = hot
    if step is not None:
        result["decode_step_with_append"] = step
    result["rk_call"] = {"us_per_call": None if rk_us is None else round(rk_us, 2), "selected": decision["selected"],
                         "entry_id": decision["entry_id"], "cache_resident": copies > 1}
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(torch, data, args.cpu_seconds)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
