"""Measure the gfx950 winners for promotion: correctness on every exact dispatch workload and paired
timing on the operator's headline workload, against the operator's declared torch fallback.

    python radeon-kernels_amd/promotion/evaluate.py --output DIR [--operators a,b] [--samples N]

Writes ``DIR/<operator>-gfx950.json`` per operator: the environment, the candidate (binding artifact
and kernel library digests, kernel source digest), one correctness record per (workload, seed) and
paired timing samples.  This plays the part of the reference's evaluation step
(benchmarks/llm_ops/evaluate.py, consumed by developer/promotion/create_operator_proposal.py:87-237):

* correctness: the public operator (which must select the native winner) against the product's
  torch fallback evaluated in fp32 on fp32 copies of the inputs ("torch_fp32_reference"), three
  seeds per workload; passes when the output is finite, the native path ran and the max absolute
  error is within the operator's bar (paged attention: fp16 2e-3, bf16 1.6e-2; KV-cache writes:
  bit-exact);
* timing, as the reference's evaluate.py:56-70,193-213 does it: the winner's entrypoint (the pack
  binding, called with the dispatch entry's launch parameters) against the fallback function on the
  same inputs; each sample is the mean over a batch of back-to-back calls bracketed by HIP events,
  the batch size calibrated to about 10 ms (at most 1000 calls) and shared by both, and the order
  of the pair alternates from sample to sample.

Run on the GPU; publish.py turns the output into proposals, evidence and pack-index records.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import math
import platform
import statistics
import sys
import time
from datetime import datetime, timezone
from pathlib import Path

PACKAGE_ROOT = Path(__file__).resolve().parents[1]
if str(PACKAGE_ROOT) not in sys.path:
    sys.path.insert(0, str(PACKAGE_ROOT))

TOLERANCE = {"fp16": 2e-3, "bf16": 1.6e-2}
SEEDS_PER_CASE = 3
WARMUPS = 20  # calls of each side before calibration (benchmarks/workloads/*-1.0.yaml: warmups 20, samples 30)
# Oracle and baseline names of benchmarks/workloads/<operator>-1.0.yaml:4-5.
METHODS = {"paged_attention_decode": "torch_fp32_paged_reference", "kv_cache_append": "torch_index_copy",
           "kv_cache_copy": "torch_snapshot_index_copy", "sdpa": "torch_fp32_explicit_attention"}
SDPA_BASELINE = "torch_scaled_dot_product_attention"  # benchmarks/workloads/sdpa-1.0.yaml:5
SDPA_TOLERANCE = 0.03  # absolute and relative, contracts/sdpa-1.0.json:23

# Headline workload per operator (the largest one: the timing the evidence reports).
HEADLINE = {
    "paged_attention_decode": "b128-gqa32x8-ragged-d128-p16-bf16",
    "kv_cache_append": "prefill-t128-mha32-d128-p32",
    "kv_cache_copy": "beam-pairs32-mha32-d128-p32",
    "sdpa": "b1-gqa32x8-s512-d128-causal",
}
# Exact paged-attention dispatch regions -> workload keys of benchmarks.workloads.
PA_WORKLOADS = {
    "b1-gqa32x8-c128-d128-p16-fp16": "c1",
    "b8-gqa32x8-c1024-d128-p16-bf16": "c2",
    "b4-mha16-c2048-d64-p32-bf16": "c3",
    "b4-gqa32x8-c1024-d256-p16-fp16": "c4",
    "b128-gqa32x8-ragged-d128-p16-bf16": "c5",
}


def sha256_bytes(data: bytes) -> str:
    return hashlib.sha256(data).hexdigest()


def sha256_file(path: Path) -> str:
    return sha256_bytes(Path(path).read_bytes())


def environment(torch) -> dict:
    from radeon_kernels.runtime.fingerprint import EnvironmentFingerprint

    fp = EnvironmentFingerprint.detect(torch_module=torch)
    return {"architecture": fp.architecture, "wavefront_size": fp.wavefront_size, "rocm_abi": fp.rocm_abi,
            "python_abi": fp.python_abi, "pytorch_version": fp.pytorch_version, "rocm": torch.version.hip,
            "device": torch.cuda.get_device_properties(0).name, "host": platform.machine()}


def candidate_record(operator: str) -> dict:
    from radeon_kernels import dispatch_plan

    artifact = {"paged_attention_decode": dispatch_plan.ARTIFACT, "kv_cache_append": dispatch_plan.KV_ARTIFACT,
                "kv_cache_copy": dispatch_plan.KV_COPY_ARTIFACT, "sdpa": dispatch_plan.SDPA_ARTIFACT}[operator]
    library, source = {"paged_attention_decode": ("librk_pa_gfx950.so", "pa_decode_gfx950.hip"),
                       "sdpa": ("librk_sdpa_gfx950.so", "sdpa_gfx950.hip")}.get(
        operator, ("librk_kv_gfx950.so", "kv_cache_gfx950.hip"))
    pack = PACKAGE_ROOT / "packs" / "gfx950"
    return {"artifact": artifact, "artifact_sha256": sha256_file(pack / artifact),
            "library_sha256": sha256_file(pack / "lib" / library),
            "source_sha256": sha256_file(PACKAGE_ROOT / "csrc" / source)}


def winner_entrypoint(record: dict):
    """The pack binding's entrypoint named by a dispatch record, with the entry's launch parameters."""

    import functools
    import importlib.util

    from radeon_kernels.runtime.resources import builtin_dispatch_registry

    manifest = builtin_dispatch_registry().get(record["operator"], "1.0")
    entry = next(e for e in manifest.entries if e.id == record["entry_id"])
    path = PACKAGE_ROOT / "packs" / "gfx950" / entry.winner.artifact
    spec = importlib.util.spec_from_file_location(path.stem, path)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return functools.partial(getattr(module, entry.winner.entrypoint), **dict(entry.launch))


def time_pair(torch, candidate, baseline, *, samples: int) -> dict:
    """Paired samples (ms per call) of the candidate and the baseline, alternating their order."""

    def one(fn, n):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(n):
            fn()
        end.record()
        end.synchronize()
        return start.elapsed_time(end) / n

    for _ in range(WARMUPS):
        candidate()
        baseline()
    torch.cuda.synchronize()
    calls = max(max(1, min(1000, math.ceil(10.0 / max(one(fn, 3), 1e-6)))) for fn in (candidate, baseline))
    c, b = [], []
    for index in range(samples):
        pairs = ((candidate, c), (baseline, b)) if index % 2 == 0 else ((baseline, b), (candidate, c))
        for fn, out in pairs:
            out.append(one(fn, calls))

    def stats(values):
        mean = statistics.fmean(values)
        return {"samples_ms": values, "median_ms": statistics.median(values),
                "coefficient_of_variation": statistics.pstdev(values) / mean}

    return {"candidate": stats(c), "baseline": stats(b), "calls_per_sample": calls}


# ---------------------------------------------------------------------------------------------
def evaluate_paged_attention(torch, samples: int) -> dict:
    import radeon_kernels as rk
    from radeon_kernels.ops.paged_attention.reference import paged_attention_decode_reference as fallback
    from benchmarks.workloads import WORKLOADS, make_inputs

    device = torch.device("cuda:0")

    def reference_fp32(data, chunk):
        outs = []
        k32, v32 = data["key_cache"].float(), data["value_cache"].float()
        for b0 in range(0, data["query"].shape[0], chunk):
            sl = slice(b0, b0 + chunk)
            outs.append(fallback(torch, data["query"][sl].float(), k32, v32, data["block_tables"][sl],
                                 data["context_lengths"][sl]))
        del k32, v32
        return torch.cat(outs)

    cases = []
    for suffix, key in PA_WORKLOADS.items():
        w = WORKLOADS[key]
        for seed in range(w.seed, w.seed + SEEDS_PER_CASE):
            data = make_inputs(w, seed=seed, device=device)
            args = (data["query"], data["key_cache"], data["value_cache"], data["block_tables"],
                    data["context_lengths"])
            sys.stderr.write(f"[case] paged_attention_decode {suffix} seed {seed}\n")
            sys.stderr.flush()
            out = rk.paged_attention_decode(*args)
            record = rk.get_last_dispatch()
            expected = reference_fp32(data, 4 if w.ragged else w.batch)
            error = float((out.float() - expected).abs().max().item())
            finite = bool(torch.isfinite(out).all().item())
            runtime_ok = record["selected"] == "native/decode_mfma"
            cases.append({"case_id": f"{suffix}-seed{seed}", "workload": suffix, "seed": seed, "dtype": w.dtype,
                          "runtime_ok": runtime_ok, "finite": finite, "max_absolute_error": error,
                          "tolerance": TOLERANCE[w.dtype], "entry_id": record["entry_id"],
                          "passed": runtime_ok and finite and error <= TOLERANCE[w.dtype]})
            del data, out, expected
            torch.cuda.empty_cache()

    w = WORKLOADS[PA_WORKLOADS[HEADLINE["paged_attention_decode"]]]
    data = make_inputs(w, device=device)
    args = (data["query"], data["key_cache"], data["value_cache"], data["block_tables"], data["context_lengths"])
    chunk = 8

    def baseline():
        for b0 in range(0, w.batch, chunk):
            sl = slice(b0, b0 + chunk)
            fallback(torch, args[0][sl], args[1], args[2], args[3][sl], args[4][sl])

    sys.stderr.write("[case] paged_attention_decode headline timing\n")
    sys.stderr.flush()
    rk.paged_attention_decode(*args)
    record = rk.get_last_dispatch()
    entrypoint = winner_entrypoint(record)
    scale = 1.0 / math.sqrt(w.head_dim)
    timing = time_pair(torch, lambda: entrypoint(*args, scale), baseline, samples=samples)
    return {"cases": cases, "timing": timing, "headline_entry_id": record["entry_id"],
            "oracle": METHODS["paged_attention_decode"],
            "baseline": f"{METHODS['paged_attention_decode']} ({chunk}-sequence chunks)"}


def evaluate_sdpa(torch, samples: int) -> dict:
    import radeon_kernels as rk
    from radeon_kernels.ops.sdpa.reference import sdpa_fallback, sdpa_reference
    from benchmarks.workloads import SDPA_CASES, SDPA_SEED, make_sdpa_inputs

    device = torch.device("cuda:0")
    cases = []
    for name, case in SDPA_CASES.items():
        scale = 1.0 / math.sqrt(case.head_dim)
        for dtype in ("fp16", "bf16"):
            for seed in range(SDPA_SEED, SDPA_SEED + SEEDS_PER_CASE):
                data = make_sdpa_inputs(case, dtype=dtype, seed=seed, device=device)
                q, k, v = data["query"], data["key"], data["value"]
                sys.stderr.write(f"[case] sdpa {name} {dtype} seed {seed}\n")
                sys.stderr.flush()
                out = rk.sdpa(q, k, v, is_causal=case.causal)
                record = rk.get_last_dispatch()
                expected = sdpa_reference(torch, q.float(), k.float(), v.float(), case.causal, scale)
                error = (out.float() - expected).abs()
                within = bool((error <= SDPA_TOLERANCE + SDPA_TOLERANCE * expected.abs()).all().item())
                finite = bool(torch.isfinite(out).all().item())
                runtime_ok = record["selected"] == "native/forward"
                cases.append({"case_id": f"{name}-{dtype}-seed{seed}", "workload": name, "seed": seed, "dtype": dtype,
                              "runtime_ok": runtime_ok, "finite": finite,
                              "max_absolute_error": float(error.max().item()), "tolerance": SDPA_TOLERANCE,
                              "entry_id": record["entry_id"], "passed": runtime_ok and finite and within})
    case = SDPA_CASES[HEADLINE["sdpa"]]
    data = make_sdpa_inputs(case, dtype="bf16", device=device)
    q, k, v = data["query"], data["key"], data["value"]
    scale = 1.0 / math.sqrt(case.head_dim)
    rk.sdpa(q, k, v, is_causal=case.causal)
    record = rk.get_last_dispatch()
    entrypoint = winner_entrypoint(record)
    sys.stderr.write("[case] sdpa headline timing\n")
    sys.stderr.flush()
    timing = time_pair(torch, lambda: entrypoint(q, k, v, case.causal, scale),
                       lambda: sdpa_fallback(torch, q, k, v, case.causal, scale), samples=samples)
    return {"cases": cases, "timing": timing, "headline_entry_id": record["entry_id"], "oracle": METHODS["sdpa"],
            "baseline": SDPA_BASELINE}


def evaluate_kv(torch, operator: str, samples: int) -> dict:
    import radeon_kernels as rk
    from radeon_kernels.ops.kv_cache.reference import kv_cache_append_reference, kv_cache_copy_reference
    from benchmarks.workloads import (APPEND_CASES, APPEND_SEED, COPY_CASES, COPY_SEED, make_append_inputs,
                                          make_copy_inputs)

    device = torch.device("cuda:0")
    append = operator == "kv_cache_append"
    cases_table, base_seed = (APPEND_CASES, APPEND_SEED) if append else (COPY_CASES, COPY_SEED)
    make = make_append_inputs if append else make_copy_inputs

    def call(data, key_cache, value_cache, native=True):
        if append:
            fn = rk.kv_cache_append if native else (lambda *a: kv_cache_append_reference(torch, *a))
            return fn(data["key"], data["value"], key_cache, value_cache, data["slot_mapping"])
        fn = rk.kv_cache_copy if native else (lambda *a: kv_cache_copy_reference(torch, *a))
        return fn(key_cache, value_cache, data["block_mapping"])

    cases = []
    for name in sorted(cases_table):
        for dtype in ("fp16", "bf16"):
            for seed in range(base_seed, base_seed + SEEDS_PER_CASE):
                data = make(name, dtype=dtype, seed=seed, device=device)
                sys.stderr.write(f"[case] {operator} {name} {dtype} seed {seed}\n")
                sys.stderr.flush()
                kc, vc = data["key_cache"].clone(), data["value_cache"].clone()
                call(data, kc, vc)
                record = rk.get_last_dispatch()
                ek, ev = data["key_cache"].float().clone(), data["value_cache"].float().clone()
                floats = dict(data)
                if append:
                    floats.update(key=data["key"].float(), value=data["value"].float())
                call(floats, ek, ev, native=False)
                error = max(float((kc.float() - ek).abs().max().item()), float((vc.float() - ev).abs().max().item()))
                finite = bool(torch.isfinite(kc).all().item() and torch.isfinite(vc).all().item())
                runtime_ok = record["selected"].startswith("native/")
                cases.append({"case_id": f"{name}-{dtype}-seed{seed}", "workload": name, "seed": seed, "dtype": dtype,
                              "runtime_ok": runtime_ok, "finite": finite, "max_absolute_error": error,
                              "tolerance": 0.0, "entry_id": record["entry_id"],
                              "passed": runtime_ok and finite and error == 0.0})
    headline = HEADLINE[operator]
    data = make(headline, dtype="bf16", device=device)
    kc, vc = data["key_cache"].clone(), data["value_cache"].clone()
    bk, bv = data["key_cache"].clone(), data["value_cache"].clone()
    sys.stderr.write(f"[case] {operator} headline timing\n")
    sys.stderr.flush()
    call(data, kc, vc)
    record = rk.get_last_dispatch()
    entrypoint = winner_entrypoint(record)
    if append:
        native = lambda: entrypoint(data["key"], data["value"], kc, vc, data["slot_mapping"])  # noqa: E731
    else:
        native = lambda: entrypoint(kc, vc, data["block_mapping"])  # noqa: E731
    timing = time_pair(torch, native, lambda: call(data, bk, bv, native=False), samples=samples)
    return {"cases": cases, "timing": timing, "headline_entry_id": record["entry_id"],
            "oracle": METHODS[operator], "baseline": METHODS[operator]}


def main(argv=None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--output", type=Path, required=True)
    parser.add_argument("--operators", default="paged_attention_decode,kv_cache_append,kv_cache_copy,sdpa")
    parser.add_argument("--samples", type=int, default=30)
    args = parser.parse_args(argv)

    import torch

    if not torch.cuda.is_available():
        print("no visible ROCm GPU", file=sys.stderr)
        return 1
    args.output.mkdir(parents=True, exist_ok=True)
    env = environment(torch)
    for operator in args.operators.split(","):
        started = time.perf_counter()
        if operator == "paged_attention_decode":
            result = evaluate_paged_attention(torch, args.samples)
        elif operator == "sdpa":
            result = evaluate_sdpa(torch, args.samples)
        else:
            result = evaluate_kv(torch, operator, args.samples)
        document = {"schema": "rk-gfx950-evaluation-1", "operator": operator, "semantic_version": "1.0",
                    "captured_at": datetime.now(timezone.utc).isoformat(), "environment": env,
                    "candidate": candidate_record(operator), **result}
        path = args.output / f"{operator}-gfx950.json"
        path.write_text(json.dumps(document, indent=1, sort_keys=True) + "\n", encoding="utf-8")
        passed = sum(case["passed"] for case in result["cases"])
        t = result["timing"]
        print(json.dumps({"operator": operator, "cases_passed": passed, "cases": len(result["cases"]),
                          "candidate_median_ms": t["candidate"]["median_ms"],
                          "baseline_median_ms": t["baseline"]["median_ms"],
                          "candidate_cv": t["candidate"]["coefficient_of_variation"],
                          "baseline_cv": t["baseline"]["coefficient_of_variation"],
                          "seconds": round(time.perf_counter() - started, 1)}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
