"""The reference's fixed quality fixture through Engine.predict on the GPU, gated against the oracle.

The reference runs the 400 typed-decision requests of benchmarks/data/typed-decisions.parquet
(2,000 decisions with gold labels) and 48 long inputs built from them through ``Engine.predict``
and gates the answers against the official SDK at FP32 (benchmarks/run.py:152-160, 205-225): mean
probability error <= 1e-3, max <= 1e-2 (act probabilities alike), decision agreement >= 99.5%,
and an exact one-sided sign test on the gold labels with p >= 0.05.  Here the same requests go
through this package's ``Engine`` (prepare -> packed slot -> HIP forward -> decode) on a seeded
ModernBERT-shaped checkpoint with the offline-trained tokenizer (no real checkpoint is available
offline), and the reference side is the FP32 oracle's logits for the same prepared items, decoded
by the same ``decode``.  Accuracy against the gold labels is at chance for random weights; the
sign test still checks that the GPU path loses no decisions the oracle gets right.
"""
import concurrent.futures as cf
import multiprocessing as mp
import os

import numpy as np
import pytest

import typed_decisions as TD
from synthetic_checkpoint import write

pytestmark = pytest.mark.gpu

_worker = {}


def _load(path):
    from safetensors.numpy import load_file

    import oracle.modernbert as MB
    from laya_cuda.laya import Laya
    adapter = Laya(path)
    cfg = MB.config(adapter)
    _worker.update(adapter=adapter, cfg=cfg, weights=MB.structured(load_file(str(path / "model.safetensors")), cfg))


def _oracle_answer(request):
    """Oracle logits of one request's prepared items, decoded as Engine.predict decodes."""
    import oracle.modernbert as MB
    state, questions = request
    adapter = _worker["adapter"]
    items = adapter.prepare(state, questions)
    logits, acts, _ = MB.forward(items, _worker["weights"], _worker["cfg"])
    padded = np.zeros((len(items), max(len(v) for v in logits)), np.float32)
    for q, v in enumerate(logits):
        padded[q, :len(v)] = v
    return adapter.decode(padded, acts, questions, items)


def _oracle_answers(path, requests):
    """The oracle side in fresh single-threaded worker processes (the FP32 forward of 2,448
    sequences takes about a minute on one core); progress is printed as results arrive."""
    workers = max(1, min(16, len(os.sched_getaffinity(0))))
    threads = {k: os.environ.get(k) for k in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS")}
    os.environ.update({k: "1" for k in threads})  # inherited by the spawned workers
    try:
        with cf.ProcessPoolExecutor(workers, mp.get_context("spawn"), initializer=_load, initargs=(path,)) as pool:
            out = []
            for answer in pool.map(_oracle_answer, requests, chunksize=4):
                out.append(answer)
                if len(out) % 100 == 0:
                    print(f"oracle: {len(out)}/{len(requests)} requests", flush=True)
            return out
    finally:
        for k, v in threads.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def test_typed_decision_fixture_passes_the_reference_gates(gpu, tmp_path):
    from laya_cuda import Engine, gates
    path, _, _ = write(tmp_path, max_len=512, head_max_len=128, layers=4, width=128, heads=2, intermediate=256,
                       head_layers=1)
    rows = TD.records()
    requests = TD.requests(rows)
    assert len(requests) == 400 and sum(len(g) for *_, g in requests) == 2000
    with Engine(str(path)) as engine:
        long = TD.long_cases(engine.adapter, rows)
        got = [engine.predict(state, questions) for _, state, questions, _ in requests]
        got_long = [engine.predict(state, questions) for _, state, questions, _ in long]
    print(f"GPU answers done; long inputs of {min(c[3] for c in long)}-{max(c[3] for c in long)} tokens", flush=True)
    want_all = _oracle_answers(path, [(s, q) for _, s, q, _ in requests] + [(s, q) for _, s, q, _ in long])
    want, want_long = want_all[:len(requests)], want_all[len(requests):]
    stats = gates.agreement(got, want, gold=[g for *_, g in requests])
    print(f"fixture: {stats}", flush=True)
    assert stats["decisions"] == 2000
    assert gates.passes(stats), gates.failures(stats)
    long_stats = gates.agreement(got_long, want_long)
    print(f"long inputs: {long_stats}", flush=True)
    assert long_stats["decisions"] == sum(len(q) for _, _, q, _ in long)
    assert gates.passes(long_stats), gates.failures(long_stats)
