"""Benchmark of the MI355X encoder forward path behind Runtime.predict (one GPU).

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--cpu-seconds 15] [--extras]

Headline workload (one JSON line on stdout): the 12-layer, d=768, 12-head, FFN 3072 post-LN
encoder with fp32 weights resident as fp16 MFMA operands (fp32 accumulate), one 512-token sequence
carrying two questions (4 and 6 options).  fp16 rather than bf16 operands: with bf16 the logits
move by 1.4e-3 from the FP32 path (over the 1e-3 bound), with fp16 by about 2e-4.  A step is one
``predict`` of that request: packed upload, hipGraph replay of the whole forward (embedding gather + LayerNorm, 12 x [QKV GEMM, attention, out GEMM,
add+LN, FFN up GEMM+GELU, FFN down GEMM, add+LN], option gather, scorer, per-question softmax,
act head) and read-back of logits and acts.

Fields:
  value / p95_ms        p50 / p95 of the forward's device time (events around the graph replay,
                        inputs already resident in HBM), ms
  predict_p50/p95_ms    the whole predict call seen by the caller (packing, H2D, replay, D2H)
  ms_per_step           wall time of the timed loop / steps
  first_ms              the first predict of the shape (slot allocation + hipGraph capture)
  roofline              the kernel with the largest share of the forward, timed live with HIP
                        events over back-to-back launches on the engine's stream
  cpu_baseline          the NumPy FP32 restatement of the same forward on this host's cores
  parity                GPU logits vs that CPU forward: max |logit error|, decisions equal
``--calibrate-copy`` first runs a 64 MiB device copy (the reference for the HBM byte counters of a
``rocprofv3 --pmc`` run).  ``--eager`` launches the forward kernel by kernel instead of replaying its hipGraph (for
profilers that cannot follow graph launches).  ``--extras`` adds the other workloads: 83- and 1,024-token latency, the 32-request ragged batch
(sequences/s) and the 24-layer d=1024 64 x 1024 batch (sequences/s and MFMA utilisation);
``--workloads`` picks a subset of them.
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "laya-cuda_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "p50/p95 predict latency (ms) at 83/512/1024 tok; seqs/sec at batch 32"
MFMA_PEAK_TFLOPS = 2500.0   # MI355X dense bf16/fp16
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E


def pct(values, q):
    return float(np.percentile(np.asarray(values, np.float64), q))


def stage_work(stage, spec, lengths):
    """Algorithmic work of ONE launch of a stage: ("mfma", FLOP) or ("hbm", bytes).

    Valid tokens only.  GEMMs 2*T*N*K; attention 4*L^2*d per sequence (QK^T and PV);
    embedding gather + LN T*(4 + 14d) + 8d bytes; residual add + LN 12*T*d bytes."""
    d, f = spec.width, spec.intermediate
    T = sum(lengths)
    if stage == "qkv":
        return "mfma", 2.0 * T * 3 * d * d
    if stage == "attn_out":
        return "mfma", 2.0 * T * d * d
    if stage in ("ffn_up", "ffn_down"):
        return "mfma", 2.0 * T * d * f
    if stage == "attention":
        return "mfma", float(sum(4 * L * L * d for L in lengths))
    if stage == "embed_norm":
        return "hbm", float(T * (4 + 14 * d) + 8 * d)
    if stage in ("attn_norm", "ffn_norm"):
        return "hbm", float(12 * T * d)
    return None, 0.0


def progress(message):
    print(f"bench: {message}", file=sys.stderr, flush=True)


def time_workload(rt, sequences, questions, steps, warmup, capture=True):
    first = time.perf_counter()
    rt.predict_sequences(sequences, questions, capture)
    first_ms = (time.perf_counter() - first) * 1e3
    for _ in range(warmup):
        rt.predict_sequences(sequences, questions, capture)
    gpu, api = [], []
    t0 = time.perf_counter()
    for _ in range(steps):
        s = time.perf_counter()
        logits, acts, metrics = rt.predict_sequences(sequences, questions, capture)
        api.append((time.perf_counter() - s) * 1e3)
        gpu.append(metrics["gpu_ms"])
    wall = time.perf_counter() - t0
    return dict(gpu=gpu, api=api, wall=wall, first_ms=first_ms, logits=logits, acts=acts, metrics=metrics)


def stage_profile(rt, spec, sequences, questions, reps):
    lengths = [len(s) for s in sequences]
    rows = []
    for name in rt.stages():
        n, layer = rt.stage_launches(name)
        if n == 0:
            continue
        ms = rt.time_stage(sequences, questions, name, layer, reps)
        bound, work = stage_work(name, spec, lengths)
        rows.append(dict(stage=name, ms=ms, launches=n, forward_ms=ms * n, bound=bound, work=work))
    return rows


def roofline(row):
    if row["bound"] == "mfma":
        achieved = row["work"] / (row["ms"] * 1e-3) / 1e12
        return {"bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / MFMA_PEAK_TFLOPS, 4), "traffic": None, "kernel": row["stage"],
                "avg_launch_us": round(row["ms"] * 1e3, 2), "work_per_launch": row["work"]}
    achieved = row["work"] / (row["ms"] * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "kernel": row["stage"],
            "avg_launch_us": round(row["ms"] * 1e3, 2), "work_per_launch": row["work"]}


def cpu_baseline(spec, weights, sequences, questions, seconds):
    """The oracle's FP32 forward of the same request, repeated for about ``seconds``."""
    import oracle.encoder as E
    try:
        from threadpoolctl import threadpool_info
        threads = max([int(i.get("num_threads", 1)) for i in threadpool_info() if i.get("user_api") == "blas"] or [1])
    except Exception:
        threads = len(os.sched_getaffinity(0))
    cfg = {"width": spec.width, "heads": spec.heads, "eps": spec.eps, "layers": spec.layers}
    w = E.structured(weights, cfg)
    out = E.forward(sequences, questions, w, cfg)  # warm-up, and the parity reference
    times = []
    start = time.perf_counter()
    while not times or (time.perf_counter() - start < seconds and len(times) < 50):
        s = time.perf_counter()
        E.forward(sequences, questions, w, cfg)
        times.append((time.perf_counter() - s) * 1e3)
    return times, threads, out


TRAFFIC = ROOT / "profiles" / "traffic.json"


def measured_traffic(stage):
    """HBM bytes per launch of ``stage`` at the 512-token workload, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE passes (profiles/traffic.json, copy-kernel calibrated), if they cover it."""
    try:
        data = json.loads(TRAFFIC.read_text())
    except (OSError, ValueError):
        return None
    entry = data.get("stages", {}).get(stage)
    return None if entry is None else entry.get("bytes_per_launch")


def calibrate_copy():
    """A plain device-to-device copy of 64 MiB, three times: the known-size reference that scales
    the FETCH_SIZE and WRITE_SIZE counters of the same profiler run."""
    import torch
    src = torch.ones(16 << 20, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def run_headline(args):
    from laya_cuda import synthetic
    from laya_cuda.runtime import Runtime

    if args.calibrate_copy:
        calibrate_copy()
        progress("copy calibration done")

    spec = synthetic.adapter("l512", mfma_dtype="float16")
    weights = synthetic.weights(spec, seed=0)
    sequences, questions = synthetic.request("l512", seed=1)
    rt = Runtime(spec, 0, 4, weights=weights)
    try:
        _sync()
        r = time_workload(rt, sequences, questions, args.steps, args.warmup, not args.eager)
        _sync()
        progress(f"l512 timed: p50 {pct(r['gpu'], 50):.4f} ms")
        rows = stage_profile(rt, spec, sequences, questions, args.stage_reps)
        progress("stage timings done")
    finally:
        rt.close()
    dominant = max((row for row in rows if row["bound"]), key=lambda row: row["forward_ms"])
    line = {
        "metric": METRIC, "value": round(pct(r["gpu"], 50), 4), "unit": "ms", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(r["wall"] * 1e3 / args.steps, 4), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic",
        "config": {"workload": "l512: 12-layer post-LN encoder d=768, 12 heads x 64, FFN 3072 GELU, vocab 50368, "
                               "batch 1 x 512 tokens, 2 questions (4 and 6 options), fp32 weights resident as "
                               "fp16 MFMA operands, fp32 accumulate", "seq_len": 512, "global_batch": 1,
                   "parallelism": "single GPU"},
        "p95_ms": round(pct(r["gpu"], 95), 4),
        "predict_p50_ms": round(pct(r["api"], 50), 4), "predict_p95_ms": round(pct(r["api"], 95), 4),
        "first_ms": round(r["first_ms"], 3), "graph_replay": not args.eager,
        "tflops_forward": round(synthetic.valid_flops(spec, [512]) / (pct(r["gpu"], 50) * 1e-3) / 1e12, 2),
        "roofline": dict(roofline(dominant), traffic=measured_traffic(dominant["stage"])),
        "stages_us_per_forward": {row["stage"]: round(row["forward_ms"] * 1e3, 2) for row in rows},
    }
    if args.cpu_seconds > 0:
        times, threads, (want, want_acts, _) = cpu_baseline(spec, weights, sequences, questions, args.cpu_seconds)
        progress(f"cpu baseline: {len(times)} forwards")
        line["cpu_baseline"] = {
            "value": round(pct(times, 50), 2), "unit": "ms", "cores": threads, "kind": "port",
            "sample": f"{len(times)} full forwards of the same 512-token request by the NumPy FP32 oracle "
                      f"(p50; BLAS threads {threads} of {len(os.sched_getaffinity(0))} host cores)"}
        worst = max(float(np.abs(r["logits"][q, :len(w)] - w).max()) for q, w in enumerate(want))
        same = all(int(np.argmax(r["logits"][q, :len(w)])) == int(np.argmax(w)) for q, w in enumerate(want))
        line["parity"] = {"max_abs_logit_err": worst, "max_abs_act_err": float(np.abs(r["acts"] - want_acts).max()),
                          "decisions_equal": same}
    else:
        line["cpu_baseline"] = None
    return line


def run_extras(args):
    from laya_cuda import synthetic
    from laya_cuda.runtime import Runtime

    extras = {}
    chosen = args.workloads.split(",") if args.workloads else None
    for name, dtype in (("l83", "float16"), ("l1024", "float16"), ("ragged32", "float16"),
                        ("b64x1024", "bfloat16")):
        if chosen and name not in chosen:
            continue
        spec = synthetic.adapter(name, mfma_dtype=dtype)
        weights = synthetic.weights(spec, seed=0, bf16=synthetic.WORKLOADS[name].get("bf16", False))
        sequences, questions = synthetic.request(name, seed=1)
        steps = args.steps if name in ("l83", "l1024") else max(5, args.steps // 20)
        rt = Runtime(spec, 0, 2, weights=weights)
        try:
            r = time_workload(rt, sequences, questions, steps, min(args.warmup, 5), not args.eager)
            rows = stage_profile(rt, spec, sequences, questions, 3 if name in ("ragged32", "b64x1024") else 20)
        finally:
            rt.close()
        progress(f"{name} timed: p50 {pct(r['gpu'], 50):.4f} ms")
        flops = synthetic.valid_flops(spec, [len(s) for s in sequences])
        p50 = pct(r["gpu"], 50)
        entry = {"p50_ms": round(p50, 4), "p95_ms": round(pct(r["gpu"], 95), 4),
                 "predict_p50_ms": round(pct(r["api"], 50), 4), "predict_p95_ms": round(pct(r["api"], 95), 4),
                 "first_ms": round(r["first_ms"], 3), "steps": steps,
                 "tflops": round(flops / (p50 * 1e-3) / 1e12, 2),
                 "mfma_frac": round(flops / (p50 * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4)}
        entry["stages_us_per_forward"] = {row["stage"]: round(row["forward_ms"] * 1e3, 2) for row in rows}
        entry["stage_frac"] = {row["stage"]: round(roofline(row)["frac"], 4) for row in rows if row["bound"]}
        if len(sequences) > 1:
            entry["seqs_per_s"] = round(len(sequences) / (p50 * 1e-3), 1)
            entry["seqs_per_s_predict"] = round(len(sequences) / (pct(r["api"], 50) * 1e-3), 1)
        extras[name] = entry
        del weights
    return extras


def _drive(submit, work, concurrency, samples, warmup):
    """Keep ``concurrency`` requests outstanding until ``samples`` complete; per-request latency is
    taken at completion (a done-callback), not when the driver polls (tools/benchmark_batching.py
    protocol of the reference)."""
    from concurrent.futures import FIRST_COMPLETED, Future, wait
    for i in range(0, warmup, concurrency):
        for f in [submit(*work[j % len(work)]) for j in range(i, min(i + concurrency, warmup))]:
            f.result()
    pending, latencies, sent = {}, [], 0
    start = time.perf_counter()
    while sent < samples or pending:
        while sent < samples and len(pending) < concurrency:
            before = time.perf_counter()
            original, done = submit(*work[sent % len(work)]), Future()

            def complete(f, finished=done):
                try:
                    f.result()
                    finished.set_result(time.perf_counter())
                except BaseException as error:  # reported by the driver
                    finished.set_exception(error)
            original.add_done_callback(complete)
            pending[done] = before
            sent += 1
        finished, _ = wait(pending, return_when=FIRST_COMPLETED)
        for f in finished:
            latencies.append((f.result() - pending.pop(f)) * 1e3)
    seconds = time.perf_counter() - start
    return {"p50_ms": round(pct(latencies, 50), 3), "p95_ms": round(pct(latencies, 95), 3),
            "p99_ms": round(pct(latencies, 99), 3), "requests_s": round(samples / seconds, 1)}


def run_batching(args):
    """Serialized Engine vs BatchEngine under bounded outstanding load on the 12-layer d=768 encoder
    (tools/benchmark_batching.py of the reference): one 2-option question per request, short
    (32-token), long (1,024-token) and alternating cases, 1 / 8 / 32 requests outstanding."""
    import shutil
    import tempfile
    from concurrent.futures import ThreadPoolExecutor

    from laya_cuda import BatchEngine, Engine, synthetic
    spec = synthetic.WORKLOADS["ragged32"]
    config = synthetic.encoder_config(spec["layers"], spec["width"], spec["heads"], spec["intermediate"],
                                      spec["vocab"], spec["positions"])
    task = dict(synthetic.task_config(spec["max_len"]), head_max_len=64)
    root = tempfile.mkdtemp(prefix="laya_batching_")
    out = {"model": "12L/768 post-LN encoder, fp16 operands, max_len 1024", "samples": args.batching_samples,
           "batch_tokens": 4096, "cases": {}}
    try:
        path = synthetic.checkpoint(root, config, task, seed=0, random_norms=False)[0]
        questions = {"0": {"type": "choice", "instructions": "Choose a topic.", "criteria": ["payment", "software"]}}
        probe = Engine(str(path), max_cached_shapes=2)
        overhead = len(probe.adapter.prepare("", questions)[0][0])
        probe.close()
        short = (" refund" * max(0, 32 - overhead), questions)
        long = (" refund" * max(0, spec["max_len"] - overhead), questions)
        cases = {"short": [short], "long": [long], "mixed": [short, long]}
        for mode in ("serial", "batch"):
            executor = ThreadPoolExecutor(1) if mode == "serial" else None
            engine = (executor.submit(Engine, str(path)).result() if executor
                      else BatchEngine(str(path), max_batch_tokens=4096))
            submit = ((lambda st, q: executor.submit(engine.predict, st, q)) if executor else engine.submit)
            try:
                for case, work in cases.items():
                    for concurrency in (1, 8, 32):
                        r = _drive(submit, work, concurrency, args.batching_samples, 20)
                        out["cases"].setdefault(case, {}).setdefault(mode, {})[str(concurrency)] = r
                        progress(f"batching {case} {mode} x{concurrency}: p50 {r['p50_ms']} ms, {r['requests_s']} req/s")
            finally:
                if executor:
                    executor.submit(engine.close).result()
                    executor.shutdown()
                else:
                    engine.close()
    finally:
        shutil.rmtree(root, ignore_errors=True)
    return out


def _sync():
    try:
        import torch
        if torch.cuda.is_available():
            torch.cuda.synchronize()
    except ImportError:
        pass


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--stage-reps", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--extras", action="store_true")
    ap.add_argument("--eager", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true")
    ap.add_argument("--batching", action="store_true",
                    help="with --extras: serialized Engine vs BatchEngine under 1/8/32 outstanding requests")
    ap.add_argument("--batching-samples", type=int, default=100)
    ap.add_argument("--workloads", default="",
                    help="with --extras: comma-separated subset of l83,l1024,ragged32,b64x1024 (default all)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the encoder path shards by request with no collective, and "
              "multi-GPU runs are not part of this build (use --gpus 1)", file=sys.stderr)
        sys.exit(2)
    line = run_headline(args)
    if args.extras:
        line["extras"] = run_extras(args)
        if args.batching:
            line["extras"]["batching"] = run_batching(args)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
