"""Engine end to end on a checkpoint directory (tokenizer, configs, safetensors): prepare on the host,
the ModernBERT forward on the GPU through liblaya_hip, decode on the host; the answers match the
oracle's logits run through the same decode (laya_cuda/engine.py:24-35 of the reference)."""
import math

import numpy as np
import pytest

from synthetic_checkpoint import write

pytestmark = pytest.mark.gpu

QUESTIONS = {
    "route": {"type": "choice", "instructions": "Choose a team for the ticket",
              "criteria": {"billing": "invoices and payment errors", "shipping": "delivery and tracking", "other": None}},
    "angry": {"type": "noul", "instructions": "Is the customer angry?"},
    "urgency": {"type": "score", "instructions": "How urgent is the ticket?",
                "criteria": ["not urgent", "urgent", "critical"]},
}
STATE = {"ticket": "the customer asks about a late delivery and wants a refund " * 4, "order": 1234}


def oracle_answers(engine, weights, spec, items):
    import oracle.modernbert as MB
    cfg = MB.config(spec)
    logits, acts, _ = MB.forward(items, MB.structured(weights, cfg), cfg)
    k = max(len(v) for v in logits)
    padded = np.zeros((len(items), k), np.float32)
    for q, v in enumerate(logits):
        padded[q, :len(v)] = v
    return engine.adapter.decode(padded, acts, QUESTIONS, items)


def test_engine_answers_match_the_oracle(gpu, tmp_path):
    from laya_cuda import Engine
    path, spec, weights = write(tmp_path, max_len=128, head_max_len=48, layers=4, head_layers=2)
    with Engine(str(path), device="cuda:0", max_cached_shapes=2) as engine:
        got = engine.predict(STATE, QUESTIONS)
        metrics = engine.last_metrics
        items = engine.adapter.prepare(STATE, QUESTIONS)
        want = oracle_answers(engine, weights, spec, items)
        again = engine.predict(STATE, QUESTIONS)
    assert got == again  # graph replay of the cached slot gives the same answers
    assert got["model"] == want["model"] and got["usage"] == want["usage"]
    assert got["answers"].keys() == want["answers"].keys()
    for qid, answer in got["answers"].items():
        ref = want["answers"][qid]
        assert answer["type"] == ref["type"]
        assert answer.get("choice") == ref.get("choice")
        assert abs(answer["confidence"] - ref["confidence"]) <= 2e-3
        assert abs(answer["action"]["act_probability"] - ref["action"]["act_probability"]) <= 2e-3
        for key, p in answer.get("probabilities", {}).items():
            assert abs(p - ref["probabilities"][key]) <= 2e-3
        if "noul" in answer:
            assert abs(answer["noul"] - ref["noul"]) <= 2e-3
        if "score" in answer:
            assert abs(answer["score"] - ref["score"]) <= 4e-3
    assert metrics["backend"] == "cuda" and metrics["precision"] == "float16"
    assert metrics["tokens_per_question"] == [len(ids) for ids, _, _ in items]
    assert metrics["cache_miss"] and metrics["graph_capture"] and metrics["gpu_ms"] > 0
    assert len(metrics["input_sha256"]) == 64 and metrics["api_ms"] >= metrics["gpu_ms"]


def test_batch_engine_answers_match_the_serial_engine(gpu, tmp_path):
    """Requests packed together by BatchEngine (laya_cuda/batching.py:74-157) get the answers the
    serial Engine gives each alone: same decisions, probabilities within 2e-3 (packing changes the
    shape class, hence GEMM tiles and summation order)."""
    from laya_cuda import BatchEngine, Engine
    path, _, _ = write(tmp_path, max_len=128, head_max_len=48, layers=4, head_layers=2)
    requests = []
    for i in range(12):
        state = {"ticket": "late delivery refund " * (1 + 3 * i), "order": i}
        qs = dict(list(QUESTIONS.items())[:1 + i % 3])
        requests.append((state, qs))
    with Engine(str(path), device="cuda:0") as serial:
        want = [serial.predict(s, q) for s, q in requests]
    with BatchEngine(str(path), max_batch_size=8, max_batch_tokens=1024, max_wait_ms=50) as batch:
        futures = [batch.submit(s, q) for s, q in requests]
        got = [f.result(timeout=120) for f in futures]
        metrics = [f.metrics for f in futures]
    assert max(m["batch_requests"] for m in metrics) > 1  # some requests really shared a pack
    for g, w in zip(got, want):
        assert g["answers"].keys() == w["answers"].keys() and g["usage"] == w["usage"]
        for qid, answer in g["answers"].items():
            ref = w["answers"][qid]
            assert answer.get("choice") == ref.get("choice")
            for key, p in answer.get("probabilities", {}).items():
                assert abs(p - ref["probabilities"][key]) <= 2e-3
            assert abs(answer["action"]["act_probability"] - ref["action"]["act_probability"]) <= 2e-3


def _saved(path):
    from safetensors.numpy import load_file
    return load_file(str(path / "model.safetensors"))


def _resave(path, tensors):
    from safetensors.numpy import save_file
    save_file({k: np.ascontiguousarray(v) for k, v in tensors.items()}, str(path / "model.safetensors"))


def test_registry_alias_loads_the_directory_and_releases_its_pool(gpu, tmp_path):
    """A registry entry with a relative path resolves against the registry's directory; the
    weights the engine holds in HBM read back bit for bit as saved (16-bit matrices as their
    rounded values); closing the engine returns every byte of its slot pool; a BatchEngine opened
    on the same alias answers as the Engine does."""
    import json

    from laya_cuda import BatchEngine, Engine
    ckpt = tmp_path / "models" / "tuned"
    write(ckpt, max_len=96, head_max_len=48, layers=2, head_layers=1)
    registry = tmp_path / "models" / "registry.json"
    registry.write_text(json.dumps({"tuned-v2": {"path": "tuned"}}))
    saved = _saved(ckpt)
    request = ({"ticket": "refund for a late delivery", "order": 7},
               {"route": QUESTIONS["route"], "angry": QUESTIONS["angry"]})
    with Engine("tuned-v2", registry=registry) as engine:
        assert engine.path == ckpt.resolve()
        for name in ("act_head.2.bias", "scorer.1.weight", "type_emb.weight"):
            np.testing.assert_array_equal(engine.runtime.weights[name].get(), saved[name])
        wqkv = engine.runtime.weights["encoder.layers.1.attn.Wqkv.weight"].get()
        np.testing.assert_array_equal(wqkv, saved["encoder.layers.1.attn.Wqkv.weight"].astype(np.float16).astype(np.float32))
        first = engine.predict(*request)
        assert engine.runtime.pool.used_bytes() > 0
    assert engine.runtime.pool.used_bytes() == 0
    with pytest.raises(RuntimeError, match="closed"):
        engine.predict(*request)
    with BatchEngine("tuned-v2", registry=registry, max_wait_ms=0) as batch:
        assert batch.submit(*request).result(60) == first


@pytest.mark.parametrize("bias,want", [((0.0, 0.0), 0.5), ((math.log(3.0), 0.0), 0.75), ((-6.0, 6.0), None)])
def test_act_output_bias_sets_the_act_probability(gpu, tmp_path, bias, want):
    """With act_head.2's weight zeroed, the act logits are its bias exactly, whatever the encoder
    computes: act_probability = softmax(bias)[0] for every question (laya.py:243-245)."""
    from laya_cuda import Engine
    ckpt = tmp_path / "act"
    write(ckpt, max_len=96, head_max_len=48, layers=2, head_layers=1)
    tensors = _saved(ckpt)
    tensors["act_head.2.weight"] = np.zeros_like(tensors["act_head.2.weight"])
    tensors["act_head.2.bias"] = np.asarray(bias, np.float32)
    _resave(ckpt, tensors)
    b = np.asarray(bias, np.float64)
    expected = round(float(np.exp(b[0] - b.max()) / np.exp(b - b.max()).sum()), 4) if want is None else want
    with Engine(str(ckpt)) as engine:
        answers = engine.predict("a payment failed twice", QUESTIONS)["answers"]
    assert [a["action"]["act_probability"] for a in answers.values()] == [expected] * len(QUESTIONS)


@pytest.mark.parametrize("name,shape", [("act_head.2.bias", (3,)), ("scorer.1.weight", (64, 32)),
                                        ("encoder.layers.0.mlp.Wi.weight", (128, 64))])
def test_checkpoint_tensor_of_the_wrong_shape_is_refused(gpu, tmp_path, name, shape):
    from laya_cuda import Engine
    ckpt = tmp_path / "bad"
    write(ckpt, max_len=96, head_max_len=48, layers=2, head_layers=1)
    tensors = _saved(ckpt)
    tensors[name] = np.zeros(shape, np.float32)
    _resave(ckpt, tensors)
    with pytest.raises(ValueError, match="Incompatible tensor shape"):
        Engine(str(ckpt))


def test_batch_engine_gates_on_a_mixed_request_stream(gpu, tmp_path):
    """A shuffled stream of requests of every question type and option count (1-6 options), with
    short, non-Latin, budget-filling and far-over-budget states, each submitted three times to a
    BatchEngine that packs them with whatever else is queued: every answer passes the accuracy
    gates (laya_cuda.gates) against the serial Engine's answer to the same request, and repeated
    submissions of one request decide alike."""
    import random

    from laya_cuda import BatchEngine, Engine, gates
    path, _, _ = write(tmp_path, max_len=256, head_max_len=64, layers=3, head_layers=2)
    states = ["", "payment failed", {"ticket": "出荷が遅れています", "lang": "ja"}, "refund please " * 40,
              {"log": ["software error"] * 300}, "ticket " * 2000]
    menus = [
        {"only": {"type": "choice", "instructions": "Pick.", "criteria": ["one"]}},
        {"topic": {"type": "choice", "instructions": "Topic?", "criteria": ["billing", "shipping", "software",
                                                                           "account", "other", "unknown"]}},
        {"urgency": QUESTIONS["urgency"], "angry": QUESTIONS["angry"]},
        QUESTIONS,
    ]
    requests = [(s, m) for s in states for m in menus]
    order = [i for i in range(len(requests)) for _ in range(3)]
    random.Random(11).shuffle(order)
    with Engine(str(path)) as serial:
        expected = [serial.predict(s, m) for s, m in requests]
    with BatchEngine(str(path), max_batch_size=12, max_batch_tokens=2048, max_wait_ms=10) as batch:
        futures = [batch.submit(*requests[i]) for i in order]
        got = [f.result(timeout=120) for f in futures]
        packed = max(f.metrics["batch_requests"] for f in futures)
    assert packed > 1
    stats = gates.agreement(got, [expected[i] for i in order])
    print(f"mixed stream: {stats}", flush=True)
    assert gates.passes(stats), gates.failures(stats)
    by_request = {}
    for i, answer in zip(order, got):
        by_request.setdefault(i, []).append({q: gates.decision(a) for q, a in answer["answers"].items()})
    assert all(all(d == seen[0] for d in seen) for seen in by_request.values())
