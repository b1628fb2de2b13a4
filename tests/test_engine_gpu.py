"""Engine end to end on a checkpoint directory (tokenizer, configs, safetensors): prepare on the host,
the ModernBERT forward on the GPU through liblaya_hip, decode on the host; the answers match the
oracle's logits run through the same decode (laya_cuda/engine.py:24-35 of the reference)."""
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


def test_custom_checkpoint_weights_registry_and_batching(gpu, tmp_path):
    """tests/test_custom_models.py of the reference on a synthetic checkpoint: a registry alias
    resolves to the directory, weights are resident and readable, the act bias decides the act
    probability, the pool is empty after close, BatchEngine answers as Engine does, and a tensor
    of the wrong shape is refused."""
    import json

    from safetensors.numpy import save_file

    from laya_cuda import BatchEngine, Engine
    custom = tmp_path / "custom-weights"
    _, spec, weights = write(custom, max_len=128, head_max_len=64, layers=1, head_layers=1)
    weights = {name: np.zeros(shape, np.float32) for name, shape in spec.weight_shapes().items()}
    registry = tmp_path / "models.json"
    registry.write_text(json.dumps({"my-finetune": {"path": "custom-weights"}}))
    queries = {"q": {"type": "choice", "instructions": "Choose", "criteria": ["yes", "no"]}}
    outputs = []
    for bias in ([-4, 4], [4, -4]):
        weights["act_head.2.bias"] = np.array(bias, np.float32)
        save_file(weights, str(custom / "model.safetensors"))
        with Engine("my-finetune", registry=registry) as engine:
            output = engine.predict("custom input", queries)
            assert engine.path == custom.resolve()
            np.testing.assert_array_equal(engine.runtime.weights["act_head.2.bias"].get(), bias)
            assert output == engine.predict("custom input", queries)
            outputs.append(output["answers"]["q"]["action"]["act_probability"])
        assert engine.runtime.pool.used_bytes() == 0
    assert outputs[0] < .001 and outputs[1] > .999
    with Engine(str(custom)) as engine:
        expected = engine.predict("custom input", queries)
    with BatchEngine("my-finetune", registry=registry) as engine:
        assert engine.submit("custom input", queries).result(60) == expected
    weights["act_head.2.bias"] = np.zeros(3, np.float32)
    save_file(weights, str(custom / "model.safetensors"))
    with pytest.raises(ValueError, match="Incompatible tensor shape"):
        Engine("my-finetune", registry=registry)


def test_batched_model_contract(gpu, tmp_path):
    """tests/test_batching_gpu.py of the reference: mixed question types, a non-Latin state, states
    past the context budget, 5- and 1-option questions, every request twice through BatchEngine;
    probabilities within 1e-3 on average and 1e-2 at most of the serial Engine's, act
    probabilities within 1e-2, decisions agreeing on >= 99.5%."""
    from laya_cuda import BatchEngine, Engine
    path, _, _ = write(tmp_path, max_len=256, head_max_len=64, layers=4, head_layers=2)
    questions = {"same": {"type": "choice", "instructions": "Choose a topic.", "criteria": ["payment", "software"]},
                 "score": {"type": "score", "instructions": "Urgency?", "criteria": ["low", "medium", "high"]},
                 "noul": {"type": "noul", "instructions": "Does it require a refund?"}}
    states = ["Please refund my payment.", "软件出现错误，请处理。", " refund" * 110, " software" * 500]
    requests = [(state, questions) for state in states]
    requests.append(("Please refund my payment.", {"same": {"type": "choice", "instructions": "Choose a topic.",
                     "criteria": ["payment", "software", "delivery", "account", "other"]}}))
    requests.append(("Please refund my payment.", {"same": {"type": "choice", "instructions": "Choose a topic.",
                     "criteria": ["only"]}}))

    def probabilities(answer):
        if "noul" in answer:
            return [answer["noul"]]
        return list(answer["probabilities"].values())

    def label(answer):
        return answer.get("choice", answer.get("score", answer.get("noul", 0) > .5))

    with Engine(str(path)) as engine:
        expected = [engine.predict(state, qs) for state, qs in requests]
    with BatchEngine(str(path), max_batch_tokens=8192, max_wait_ms=5) as engine:
        futures = [engine.submit(state, qs) for state, qs in requests * 2]
        differences, agreement = [], []
        for i, future in enumerate(futures):
            actual, reference = future.result(120), expected[i % len(requests)]
            assert actual["usage"] == reference["usage"]
            assert list(actual["answers"]) == list(reference["answers"])
            for key, a in actual["answers"].items():
                b = reference["answers"][key]
                differences.extend(np.abs(np.array(probabilities(a)) - probabilities(b)))
                agreement.append(label(a) == label(b) if "score" not in a else abs(a["score"] - b["score"]) <= .01)
                assert abs(a["action"]["act_probability"] - b["action"]["act_probability"]) <= .01
    assert np.isfinite(differences).all()
    assert np.mean(differences) <= .001 and max(differences) <= .01
    assert np.mean(agreement) >= .995
