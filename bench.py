"""Benchmark of the MI355X encoder forward path behind Runtime.predict (one GPU).

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--cpu-seconds 15] [--only NAMES] [--eager]

One JSON line on stdout.  Headline (`value`): the 512-token workload - the 12-layer, d=768,
12-head, FFN 3072 post-LN encoder with fp32 weights resident as fp16 MFMA operands (fp32
accumulate), one 512-token sequence carrying two questions (4 and 6 options).  fp16 rather than
bf16 operands: with bf16 the logits move by 1.4e-3 from the FP32 path (over the 1e-3 bound), with
fp16 by about 2e-4.  A step is one `predict` of the request: packed upload, hipGraph replay of the
whole forward, read-back of logits and acts.

Every workload of the metric is measured in the same run, under `workloads`:
  l83        same encoder, 83 tokens, one 4-option question              p50/p95 latency
  l1024      12L/768, 250,002-row vocabulary, 1,024 Zipf tokens, 3x5      p50/p95 latency
  ragged32   32 requests of 40-900 tokens, 1-5 questions of 4-77 options  sequences/s
  b64x1024   24L/1024, 16 heads, bf16-valued weights as fp16 operands, 64 x 1,024 tokens, 8 options
                                                                         sequences/s, MFMA fraction
and three host-inclusive measurements:
  engine_predict_l512  Engine.predict on a synthetic checkpoint with a tokenizer: tokenise, pack,
                       forward, decode (the reference's definition of predict latency)
  batching             Engine serialised behind a lock vs BatchEngine, closed-loop clients
                       (1/8/32 in flight), latency percentiles, requests/s, slot-cache misses
  modernbert_base_predict  Engine.predict at 83/512/1,024 tokens on a ModernBERT-base-shaped
                       checkpoint (22L/768, GeGLU, windows, RoPE, one head layer; random weights):
                       the architecture family of the real Laya checkpoints

Per workload: p50/p95 of the forward's device time (events around the graph replay; inputs
resident in HBM) and of the whole predict call (packing, H2D, replay, D2H); first_ms (slot
allocation + graph capture); per-stage device time per forward, each stage timed where it runs
(every kernel of the stage inside eager forwards records its own start and end events, the
interval a kernel trace reports); `roofline` of the stage with the
largest share; `cpu_baseline` (the NumPy FP32 oracle of the same forward on this host's cores) and
`parity` (GPU logits against that CPU forward).
"""
import argparse
import json
import os
import shutil
import sys
import tempfile
import threading
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "laya-cuda_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "p50/p95 predict latency (ms) at 83/512/1024 tok; seqs/sec at batch 32"
MFMA_PEAK_TFLOPS = 2500.0   # MI355X dense bf16/fp16
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
TRAFFIC = ROOT / "profiles" / "traffic.json"

# name: (MFMA operand type, text of the workload)
WORKLOADS = {
    "l512": ("float16", "12-layer post-LN encoder d=768, 12 heads x 64, FFN 3072 GELU, vocab 50368, batch 1 x 512 "
                        "tokens, 2 questions (4 and 6 options), fp32 weights resident as fp16 MFMA operands, fp32 "
                        "accumulate"),
    "l83": ("float16", "same 12L/768 encoder, batch 1 x 83 tokens, one 4-option question, fp16 operands"),
    "l1024": ("float16", "12L/768 encoder, vocab 250,002 (768 MB fp32 table), 1,024 positions, batch 1 x 1,024 "
                         "Zipf(1.1) tokens, 3 questions x 5 options, fp16 operands"),
    "ragged32": ("float16", "12L/768 encoder, 32 requests of U{40..900} tokens packed back to back, 1-5 questions "
                            "of 4-77 options each, fp16 operands"),
    "b64x1024": ("float16", "24-layer post-LN encoder d=1024, 16 heads x 64, FFN 4096 GELU, N(0, 0.02) bf16-valued "
                            "weights held exactly as fp16 MFMA operands (bf16 operands cannot meet the 1e-3 logit "
                            "bound on this model: 2.85e-3 in a CPU emulation of the rounding points, fp16 2.8e-4), "
                            "fp32 accumulate, 64 x 1,024 dense tokens, one 8-option question per sequence"),
}


def pct(values, q):
    return float(np.percentile(np.asarray(values, np.float64), q))


def progress(message):
    print(f"bench: {message}", file=sys.stderr, flush=True)


def stage_work(stage, spec, lengths):
    """Algorithmic work of ONE launch of a stage: ("mfma", FLOP) or ("hbm", bytes), valid tokens only.
    GEMMs 2*T*N*K; attention 4*L^2*d per sequence (QK^T and PV); embedding gather + LN
    T*(4 + 14d) + 8d bytes; residual add + LN 12*T*d bytes."""
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


def blas_threads():
    try:
        from threadpoolctl import threadpool_info
        return max([int(i.get("num_threads", 1)) for i in threadpool_info() if i.get("user_api") == "blas"] or [1])
    except Exception:
        return len(os.sched_getaffinity(0))


def measured_traffic(workload, stage):
    """HBM bytes per launch of `stage` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes
    (copy-kernel calibrated), when they cover this workload and stage."""
    try:
        data = json.loads(TRAFFIC.read_text())
    except (OSError, ValueError):
        return None
    entry = data.get(workload, {}).get("stages", {}).get(stage)
    return None if entry is None else entry.get("bytes_per_launch")


def time_predict(rt, sequences, questions, steps, warmup, capture):
    start = time.perf_counter()
    rt.predict_sequences(sequences, questions, capture)
    first_ms = (time.perf_counter() - start) * 1e3
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
    """Per stage: average device time of one launch where it runs (start/end events of every
    kernel of the stage inside `reps` eager forwards), launches per forward and algorithmic work."""
    lengths = [len(s) for s in sequences]
    rows = []
    for name in rt.stages():
        n, _ = rt.stage_launches(name)
        if n == 0:
            continue
        ms = rt.time_stage(sequences, questions, name, -1, reps)
        bound, work = stage_work(name, spec, lengths)
        rows.append(dict(stage=name, ms=ms, launches=n, forward_ms=ms * n, bound=bound, work=work))
    return rows


def roofline(row, workload):
    rate = row["work"] / (row["ms"] * 1e-3)
    if row["bound"] == "mfma":
        achieved, peak, unit = rate / 1e12, MFMA_PEAK_TFLOPS, "TFLOP/s"
    else:
        achieved, peak, unit = rate / 1e9, HBM_PEAK_GBS, "GB/s"
    return {"bound": row["bound"], "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": measured_traffic(workload, row["stage"]),
            "kernel": row["stage"], "avg_launch_us": round(row["ms"] * 1e3, 3), "work_per_launch": row["work"],
            "timing": "start/end events of every kernel of the stage inside eager forwards (hipExtLaunchKernel, engine stream)"}


def oracle_forward(spec, weights, sequences, questions):
    import oracle.encoder as E
    cfg = {"width": spec.width, "heads": spec.heads, "eps": spec.eps, "layers": spec.layers}
    w = E.structured(weights, cfg)
    return lambda: E.forward(sequences, questions, w, cfg)


def cpu_baseline(run, seconds, most=50):
    """Time `run` (the oracle's FP32 forward) for about `seconds` (at least once); returns
    (times in ms, the last output).  The first call is a warm-up unless it alone took over 2 s
    (then it is the first sample)."""
    s = time.perf_counter()
    out = run()
    first = (time.perf_counter() - s) * 1e3
    times = [first] if first > 2000 else []
    start = time.perf_counter()
    while not times or (time.perf_counter() - start < seconds and len(times) < most):
        s = time.perf_counter()
        out = run()
        times.append((time.perf_counter() - s) * 1e3)
    return times, out


def parity(got_logits, got_acts, want_logits, want_acts):
    worst = max(float(np.abs(got_logits[q, :len(w)] - w).max()) for q, w in enumerate(want_logits))
    flips = [q for q, w in enumerate(want_logits) if int(np.argmax(got_logits[q, :len(w)])) != int(np.argmax(w))]
    return {"max_abs_logit_err": worst, "max_abs_act_err": float(np.abs(got_acts - want_acts).max()),
            "questions": len(want_logits), "decisions_differing": flips}


def run_workload(name, args):
    """Timing, stage profile, roofline, CPU baseline and parity of one workload."""
    from laya_cuda import synthetic
    from laya_cuda.runtime import Runtime

    dtype, text = WORKLOADS[name]
    spec = synthetic.adapter(name, mfma_dtype=dtype)
    weights = synthetic.weights(spec, seed=0, bf16=synthetic.WORKLOADS[name].get("bf16", False))
    sequences, questions = synthetic.request(name, seed=1)
    lengths = [len(s) for s in sequences]
    heavy = name in ("ragged32", "b64x1024")
    steps = args.steps if not heavy else max(5, args.steps // 2) if name == "ragged32" else max(3, args.steps // 4)
    warmup = args.warmup if not heavy else min(args.warmup, 3)
    rt = Runtime(spec, 0, 2, weights=weights)
    try:
        r = time_predict(rt, sequences, questions, steps, warmup, not args.eager)
        progress(f"{name}: p50 {pct(r['gpu'], 50):.4f} ms device, {pct(r['api'], 50):.4f} ms predict")
        rows = stage_profile(rt, spec, sequences, questions, 2 if heavy else args.stage_reps)
        progress(f"{name}: stage timings done")
    finally:
        rt.close()
    p50 = pct(r["gpu"], 50)
    flops = synthetic.valid_flops(spec, lengths)
    dominant = max((row for row in rows if row["bound"]), key=lambda row: row["forward_ms"])
    out = {"workload": text, "dtype": "f16" if dtype == "float16" else "bf16", "steps": steps, "warmup": warmup,
           "p50_ms": round(p50, 4), "p95_ms": round(pct(r["gpu"], 95), 4),
           "predict_p50_ms": round(pct(r["api"], 50), 4), "predict_p95_ms": round(pct(r["api"], 95), 4),
           "ms_per_step": round(r["wall"] * 1e3 / steps, 4), "first_ms": round(r["first_ms"], 3),
           "graph_replay": bool(r["metrics"]["graph_replay"]), "shape": list(r["metrics"]["shape"]),
           "valid_tokens": int(sum(lengths)), "gflop_forward": round(flops / 1e9, 2),
           "tflops_forward": round(flops / (p50 * 1e-3) / 1e12, 2),
           "mfma_frac_forward": round(flops / (p50 * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4),
           "roofline": roofline(dominant, name),
           "stages_us_per_forward": {row["stage"]: round(row["forward_ms"] * 1e3, 2) for row in rows},
           "stage_frac": {row["stage"]: roofline(row, name)["frac"] for row in rows if row["bound"]}}
    if len(sequences) > 1:
        out["seqs_per_s"] = round(len(sequences) / (p50 * 1e-3), 1)
        out["seqs_per_s_predict"] = round(len(sequences) / (pct(r["api"], 50) * 1e-3), 1)
    if args.cpu_seconds > 0:
        # The oracle on the whole request; for the 64-sequence batch on its first sequence only
        # (sequences are independent), scaled to the batch.
        picks = [0] if name == "b64x1024" else list(range(len(sequences)))
        sub_q = [(picks.index(s), m, k) for s, m, k in questions if s in picks]
        run = oracle_forward(spec, weights, [sequences[i] for i in picks], sub_q)
        budget = args.cpu_seconds if name == "l512" else min(args.cpu_seconds, 8.0)
        times, (want, want_acts, _) = cpu_baseline(run, budget)
        cpu_ms = pct(times, 50)
        cores = blas_threads()
        qrows = [q for q, (s, _, _) in enumerate(questions) if s in picks]
        if name == "b64x1024":
            out["cpu_baseline"] = {"value": round(1e3 / cpu_ms, 3), "unit": "seq/s", "cores": cores, "kind": "port",
                                   "sample": f"{len(times)} oracle FP32 forwards of sequence 0 (1,024 tokens, 24 "
                                             f"layers; p50 {cpu_ms:.0f} ms) scaled to the 64-sequence batch; BLAS "
                                             f"threads {cores} of {len(os.sched_getaffinity(0))} host cores"}
        elif len(sequences) > 1:
            out["cpu_baseline"] = {"value": round(len(sequences) / (cpu_ms * 1e-3), 3), "unit": "seq/s",
                                   "cores": cores, "kind": "port",
                                   "sample": f"{len(times)} oracle FP32 forwards of the whole request (p50 "
                                             f"{cpu_ms:.0f} ms); BLAS threads {cores} of "
                                             f"{len(os.sched_getaffinity(0))} host cores"}
        else:
            out["cpu_baseline"] = {"value": round(cpu_ms, 3), "unit": "ms", "cores": cores, "kind": "port",
                                   "sample": f"{len(times)} oracle FP32 forwards of the same request (p50); BLAS "
                                             f"threads {cores} of {len(os.sched_getaffinity(0))} host cores"}
        out["parity"] = parity(r["logits"][qrows], r["acts"][qrows], want, want_acts)
        progress(f"{name}: cpu baseline {len(times)} forwards")
    else:
        out["cpu_baseline"] = None
    return out


def synthetic_checkpoint(root, layers=12, width=768, heads=12, intermediate=3072, vocab=50368, max_len=512):
    from laya_cuda import synthetic
    config = synthetic.encoder_config(layers, width, heads, intermediate, vocab, max_len)
    task = dict(synthetic.task_config(max_len), head_max_len=64)
    return synthetic.checkpoint(root, config, task, seed=0, random_norms=False)[0]


QUESTION = {"0": {"type": "choice", "instructions": "Choose a team for billing questions.",
                  "criteria": ["payment", "software", "delivery", "other"]}}


def run_engine_predict(path, args):
    """Engine.predict at 512 tokens: the request is tokenised, packed, run and decoded on every call
    (the reference measures predict this way, including tokenisation and decode)."""
    from laya_cuda import Engine
    with Engine(str(path), max_cached_shapes=4) as engine:
        state = "the customer asks about a late delivery and wants a refund " * 80
        items = engine.adapter.prepare(state, QUESTION)
        tokens = [len(i[0]) for i in items]
        for _ in range(args.warmup + 1):
            engine.predict(state, QUESTION)
        api, gpu = [], []
        for _ in range(args.steps):
            s = time.perf_counter()
            engine.predict(state, QUESTION)
            api.append((time.perf_counter() - s) * 1e3)
            gpu.append(engine.last_metrics["gpu_ms"])
        prep = []
        for _ in range(args.steps):
            s = time.perf_counter()
            engine.adapter.prepare(state, QUESTION)
            prep.append((time.perf_counter() - s) * 1e3)
    return {"model": "12L/768 post-LN encoder, fp16 operands, synthetic checkpoint with a BPE tokenizer trained "
                     "offline; one 4-option choice question", "tokens_per_question": tokens, "steps": args.steps,
            "p50_ms": round(pct(api, 50), 4), "p95_ms": round(pct(api, 95), 4),
            "gpu_p50_ms": round(pct(gpu, 50), 4), "prepare_p50_ms": round(pct(prep, 50), 4)}


def run_modernbert_predict(path, args):
    """Engine.predict on a ModernBERT-base-shaped checkpoint at 83, 512 and 1,024 tokens: 22 layers,
    d=768, 12 heads, GeGLU 1152, RoPE, global attention every third layer and +-64 windows on the
    others, one head layer, random weights, the offline BPE tokenizer; every call tokenises, packs,
    runs and decodes.  Real Laya checkpoints are ModernBERT/mmBERT encoders whose dimensions the
    reference does not record, and its published predict latencies (README.md:13-16) are for those:
    context for them, not a like-for-like comparison."""
    from laya_cuda import Engine
    out = {"model": "ModernBERT-base-shaped: 22L/768, 12 heads, GeGLU 1152, global every 3rd layer, +-64 windows, "
                    "RoPE 160000/10000, one head layer, fp16 operands; random weights, BPE tokenizer trained "
                    "offline; one 4-option choice question", "steps": args.steps}
    with Engine(str(path), max_cached_shapes=4) as engine:
        overhead = len(engine.adapter.prepare("", QUESTION)[0][0])
        for target in (83, 512, 1024):
            state = " refund" * max(1, target - overhead)
            tokens = len(engine.adapter.prepare(state, QUESTION)[0][0])
            for _ in range(args.warmup + 1):
                engine.predict(state, QUESTION)
            api, gpu = [], []
            for _ in range(args.steps):
                s = time.perf_counter()
                engine.predict(state, QUESTION)
                api.append((time.perf_counter() - s) * 1e3)
                gpu.append(engine.last_metrics["gpu_ms"])
            out[f"tokens_{target}"] = {"tokens": tokens, "p50_ms": round(pct(api, 50), 4),
                                       "p95_ms": round(pct(api, 95), 4), "gpu_p50_ms": round(pct(gpu, 50), 4)}
            progress(f"modernbert-base {tokens} tokens: predict p50 {out[f'tokens_{target}']['p50_ms']} ms")
    return out


def closed_loop(call, requests, clients, per_client):
    """`clients` threads, each issuing `per_client` requests one after another (a request waits
    for the previous answer of its thread): per-request latency percentiles and requests/s."""
    latencies, errors = [], []
    lock = threading.Lock()

    def client(c):
        mine = []
        for i in range(per_client):
            state, questions = requests[(c + i) % len(requests)]
            s = time.perf_counter()
            try:
                call(state, questions)
            except Exception as error:  # reported, not raised, so the run finishes
                errors.append(repr(error))
            mine.append((time.perf_counter() - s) * 1e3)
        with lock:
            latencies.extend(mine)

    threads = [threading.Thread(target=client, args=(c,)) for c in range(clients)]
    start = time.perf_counter()
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    seconds = time.perf_counter() - start
    return {"p50_ms": round(pct(latencies, 50), 3), "p95_ms": round(pct(latencies, 95), 3),
            "p99_ms": round(pct(latencies, 99), 3), "requests_s": round(len(latencies) / seconds, 1),
            "requests": len(latencies), "errors": errors[:3]}


def run_batching(path, args):
    """A serialised Engine (one lock, as a single-owner service would hold it) against BatchEngine,
    with 1, 8 and 32 closed-loop clients on short (32-token), long (512-token) and alternating
    requests.  BatchEngine keeps at most 4 shape slots, so the mixed case also reports how often a
    pack needed a new slot (graph capture) under that LRU bound."""
    from laya_cuda import BatchEngine, Engine
    probe = Engine(str(path), max_cached_shapes=1)
    overhead = len(probe.adapter.prepare("", QUESTION)[0][0])
    probe.close()
    short = (" refund" * max(1, 32 - overhead), QUESTION)
    long = ("the customer asks about a late delivery and wants a refund " * 80, QUESTION)
    cases = {"short": [short], "long": [long], "mixed": [short, long]}
    per = max(8, args.batching_requests)
    out = {"requests_per_client": per, "max_batch_tokens": 8192, "max_cached_shapes": 4, "cases": {}}
    engine = Engine(str(path), max_cached_shapes=4)
    guard = threading.Lock()

    def serial(state, questions):
        with guard:
            return engine.predict(state, questions)
    try:
        for case, work in cases.items():
            for clients in (1, 8, 32):
                serial(*work[0])
                r = closed_loop(serial, work, clients, per if clients < 32 else max(4, per // 2))
                out["cases"].setdefault(case, {}).setdefault("serial", {})[str(clients)] = r
    finally:
        engine.close()
    misses = {"packs": 0, "cache_miss": 0}
    with BatchEngine(str(path), max_batch_size=16, max_batch_tokens=8192, max_wait_ms=1,
                     max_cached_shapes=4) as batch:
        def batched(state, questions):
            future = batch.submit(state, questions)
            result = future.result(120)
            with guard:
                misses["packs"] += 1
                misses["cache_miss"] += bool(future.metrics.get("cache_miss"))
            return result
        for case, work in cases.items():
            for clients in (1, 8, 32):
                batched(*work[0])
                r = closed_loop(batched, work, clients, per if clients < 32 else max(4, per // 2))
                out["cases"].setdefault(case, {}).setdefault("batch", {})[str(clients)] = r
                progress(f"batching {case} x{clients}: batch p50 {r['p50_ms']} ms {r['requests_s']} req/s, serial "
                         f"{out['cases'][case]['serial'][str(clients)]['requests_s']} req/s")
    out["batch_requests_with_new_slot"] = misses
    return out


# ---- the reference's latency suite (benchmarks/run.py:52-73, 127-151, 279-297) ----
SUITE_QUESTION = {"type": "choice", "instructions": "Pick a topic.", "criteria": ["finance", "software"]}
FILLER = " refund"


def latency_cases(adapter):
    """(name, state, questions) of the reference's latency cases: every length of 32-1,024 tokens that
    fits max_len x 1, 5 and 10 questions, built from a repeated one-token word (the reference repeats
    " investigation", one token for its checkpoints' tokenizers; " refund" is one for the offline
    tokenizer) and checked to give exactly that many tokens; one question at 127, 129 and max_len - 1 tokens (the span boundaries); five
    questions of different instruction lengths over a short state."""
    def tokens(state, questions):
        return len(adapter.prepare(state, questions)[0][0])

    out = []
    for length in (32, 64, 128, 256, 512, 768, 1024):
        if length > adapter.max_len:
            continue
        for count in (1, 5, 10):
            questions = {str(i): SUITE_QUESTION for i in range(count)}
            state = FILLER * max(0, length - tokens("", questions))
            if tokens(state, questions) != length:
                raise RuntimeError(f"latency case l{length}-q{count} has {tokens(state, questions)} tokens")
            out.append((f"l{length}-q{count}", state, questions))
    single = {"0": SUITE_QUESTION}
    for length in (127, 129, adapter.max_len - 1):
        out.append((f"boundary-l{length}", FILLER * (length - tokens("", single)), single))
    mixed = {str(i): {"type": "choice", "instructions": "Choose. " + "Different detail. " * i, "criteria": ["yes", "no"]}
             for i in range(5)}
    out.append(("mixed-lengths", "A support case about a payment.", mixed))
    return out


def suite_worker(args):
    """One round of the suite in this fresh process: every latency case (first request, warm-up,
    timed samples: p50/p95/p99 of Engine.predict and of the device time), in forward order on even
    rounds and reversed on odd ones, then the 400 typed-decision requests of the fixed quality
    fixture once each in fixture order (p50/p95/p99, and how many needed a new shape slot under
    the default 16-slot cache)."""
    import gzip
    from laya_cuda import Engine
    result = {"round": args.suite_round, "cases": {}}
    start = time.perf_counter()
    with Engine(args.suite_checkpoint) as engine:
        result["load_ms"] = round((time.perf_counter() - start) * 1e3, 1)
        cases = latency_cases(engine.adapter)
        for name, state, questions in (cases if args.suite_round % 2 == 0 else cases[::-1]):
            cold = time.perf_counter()
            engine.predict(state, questions)
            first_ms = (time.perf_counter() - cold) * 1e3
            first = engine.last_metrics
            for _ in range(args.warmup):
                engine.predict(state, questions)
            api, gpu = [], []
            for _ in range(args.steps):
                s = time.perf_counter()
                engine.predict(state, questions)
                api.append((time.perf_counter() - s) * 1e3)
                gpu.append(engine.last_metrics["gpu_ms"])
            result["cases"][name] = {
                "tokens": engine.last_metrics["tokens_per_question"][0], "questions": len(questions),
                "first_ms": round(first_ms, 3), "first_cache_miss": bool(first["cache_miss"]),
                "p50_ms": round(pct(api, 50), 4), "p95_ms": round(pct(api, 95), 4), "p99_ms": round(pct(api, 99), 4),
                "gpu_p50_ms": round(pct(gpu, 50), 4), "questions_per_s": round(len(questions) * 1e3 / np.mean(api), 1)}
        fixture = json.loads(gzip.decompress((ROOT / "tests" / "golden" / "typed_decisions.json.gz").read_bytes()))
        api, gpu, cold = [], [], 0
        for row in fixture["records"]:
            state, questions = json.loads(row["state"]), json.loads(row["questions"])
            s = time.perf_counter()
            engine.predict(state, questions)
            api.append((time.perf_counter() - s) * 1e3)
            gpu.append(engine.last_metrics["gpu_ms"])
            cold += bool(engine.last_metrics["cache_miss"])
        result["fixture"] = {"requests": len(api), "p50_ms": round(pct(api, 50), 4), "p95_ms": round(pct(api, 95), 4),
                             "p99_ms": round(pct(api, 99), 4), "gpu_p50_ms": round(pct(gpu, 50), 4),
                             "cold_shape_requests": cold}
    Path(args.suite_out).write_text(json.dumps(result))


def modernbert_base_checkpoint(root):
    """ModernBERT-base-shaped checkpoint (22L/768, 12 heads, GeGLU 1152, max_len 1,024, one head layer)."""
    from laya_cuda import synthetic
    config = synthetic.modernbert_config(22, 768, 12, 1152, 50368, 8192)
    task = dict(synthetic.task_config(1024), head_layers=1, head_max_len=64)
    return synthetic.checkpoint(root, config, task, seed=0, random_norms=False)[0]


def run_latency_suite(path, args):
    """Three rounds of the suite, each in a fresh child process started one after another before
    this process touches the GPU, on a ModernBERT-base-shaped checkpoint with max_len 1,024 (the
    architecture family of the real Laya checkpoints; random weights, offline BPE tokenizer).  Per
    case the rounds' p50/p95/p99 and first-request times are listed, with the median over rounds;
    the fixture's 400 requests give the mixed-request p50/p95/p99 and cold-shape counts."""
    import subprocess
    root = tempfile.mkdtemp(prefix="laya_suite_")
    rounds = []
    try:
        for r in range(3):
            out = Path(root) / f"round{r}.json"
            cmd = [sys.executable, str(ROOT / "bench.py"), "--suite-worker", "--suite-round", str(r),
                   "--suite-checkpoint", str(path), "--suite-out", str(out), "--steps", str(args.steps),
                   "--warmup", str(args.warmup)]
            subprocess.run(cmd, check=True, timeout=600)
            rounds.append(json.loads(out.read_text()))
            progress(f"latency suite round {r}: fixture p50/p95/p99 {rounds[-1]['fixture']['p50_ms']}/"
                     f"{rounds[-1]['fixture']['p95_ms']}/{rounds[-1]['fixture']['p99_ms']} ms, "
                     f"{rounds[-1]['fixture']['cold_shape_requests']} cold")
    finally:
        shutil.rmtree(root, ignore_errors=True)
    cases = {}
    for name in rounds[0]["cases"]:
        per = [rd["cases"][name] for rd in rounds]
        cases[name] = {"tokens": per[0]["tokens"], "questions": per[0]["questions"],
                       **{k: [p[k] for p in per] for k in ("p50_ms", "p95_ms", "p99_ms", "first_ms", "gpu_p50_ms")},
                       "median_p50_ms": round(float(np.median([p["p50_ms"] for p in per])), 4),
                       "median_p99_ms": round(float(np.median([p["p99_ms"] for p in per])), 4)}
    fixture = [rd["fixture"] for rd in rounds]
    return {"model": "ModernBERT-base-shaped: 22L/768, 12 heads, GeGLU 1152, global every 3rd layer, +-64 windows, "
                     "max_len 1,024, one head layer, fp16 operands; random weights, offline BPE tokenizer",
            "protocol": f"3 rounds in fresh processes (case order reversed on odd rounds), {args.warmup} warm-ups "
                        f"and {args.steps} samples per case (the reference: 20 and 200)",
            "load_ms": [rd["load_ms"] for rd in rounds], "cases": cases,
            "cases_first_request_cold": sum(c["first_cache_miss"] for rd in rounds for c in rd["cases"].values()),
            "fixture_requests": {k: [f[k] for f in fixture] for k in fixture[0]}}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--stage-reps", type=int, default=10, help="eager forwards per stage for the stage timings")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="oracle time budget of the headline (0: none)")
    ap.add_argument("--only", default="", help="comma-separated subset of " + ",".join(
        list(WORKLOADS) + ["engine", "batching", "modernbert", "suite"]) + " (default all; l512 is always the headline)")
    ap.add_argument("--batching-requests", type=int, default=24, help="requests per closed-loop client")
    ap.add_argument("--eager", action="store_true", help="launch kernel by kernel instead of replaying hipGraphs")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run a 64 MiB device copy (the reference size for HBM byte counters)")
    ap.add_argument("--suite-worker", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--suite-round", type=int, default=0, help=argparse.SUPPRESS)
    ap.add_argument("--suite-checkpoint", help=argparse.SUPPRESS)
    ap.add_argument("--suite-out", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.suite_worker:
        return suite_worker(args)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the encoder path shards by request with no collective, and "
              "multi-GPU runs are not implemented (use --gpus 1)", file=sys.stderr)
        sys.exit(2)
    chosen = set(args.only.split(",")) if args.only else set(WORKLOADS) | {"engine", "batching", "modernbert", "suite"}
    mb_root = tempfile.mkdtemp(prefix="laya_bench_mb_")
    mb_path = modernbert_base_checkpoint(mb_root) if chosen & {"suite", "modernbert"} else None
    # The latency suite's rounds run in fresh child processes, before this process touches the GPU.
    suite = run_latency_suite(mb_path, args) if "suite" in chosen else None
    if args.calibrate_copy:
        import torch
        src = torch.ones(16 << 20, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        progress("copy calibration done")

    head = run_workload("l512", args)
    line = {"metric": METRIC, "value": head["p50_ms"], "unit": "ms", "n_gpus": 1, "steps": head["steps"],
            "warmup": head["warmup"], "ms_per_step": head["ms_per_step"], "higher_is_better": False,
            "scaling": "weak", "vs_baseline": None, "dtype": head["dtype"], "data": "synthetic",
            "config": {"workload": "l512: " + head["workload"], "seq_len": 512, "global_batch": 1,
                       "parallelism": "single GPU"}}
    for key in ("p95_ms", "predict_p50_ms", "predict_p95_ms", "first_ms", "graph_replay", "tflops_forward",
                "roofline", "stages_us_per_forward", "cpu_baseline", "parity"):
        if key in head:
            line[key] = head[key]
    line["workloads"] = {}
    for name in ("l83", "l1024", "ragged32", "b64x1024"):
        if name in chosen:
            line["workloads"][name] = run_workload(name, args)
    if chosen & {"engine", "batching"}:
        root = tempfile.mkdtemp(prefix="laya_bench_")
        try:
            path = synthetic_checkpoint(root)
            if "engine" in chosen:
                line["engine_predict_l512"] = run_engine_predict(path, args)
                progress(f"engine predict p50 {line['engine_predict_l512']['p50_ms']} ms")
            if "batching" in chosen:
                line["batching"] = run_batching(path, args)
        finally:
            shutil.rmtree(root, ignore_errors=True)
    if "modernbert" in chosen:
        line["modernbert_base_predict"] = run_modernbert_predict(mb_path, args)
    shutil.rmtree(mb_root, ignore_errors=True)
    if suite is not None:
        line["latency_suite"] = suite
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
